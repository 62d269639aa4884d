/* lg_common.h -- shared device helpers of the gfx950 decode path. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/ligguf_hip.h"

/* GGUF block byte sizes and field offsets (fast/lil_gguf.h:64-119) */
#define LG_QK8_0 32
#define LG_QK_K 256
#define LG_BS_Q8_0 34
#define LG_BS_Q1_0 6
#define LG_BS_Q1_G 18
#define LG_BS_Q2_K 84
#define LG_BS_Q3_K 110
#define LG_BS_Q4_K 144
#define LG_BS_Q5_K 176
#define LG_BS_Q6_K 210
#define LG_BS_Q8_K 292

#define LG_WAVE 64

/* record an error message for the calling host thread / context */
void lg_set_error(const char* fmt, ...);
const char* lg_get_thread_error(void);

#define LG_HIP_CHECK(expr)                                                                 \
    do {                                                                                   \
        hipError_t e__ = (expr);                                                           \
        if (e__ != hipSuccess) {                                                           \
            lg_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e__), __FILE__, \
                         __LINE__);                                                        \
            return LG_ERR_HIP;                                                             \
        }                                                                                  \
    } while (0)

/* ---- device helpers ---- */

__device__ __forceinline__ float lg_h2f(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

/* IEEE round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 in the default mode) */
__device__ __forceinline__ uint16_t lg_f2h(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

/* unaligned little-endian loads (gfx950 serves unaligned global dword loads) */
template <typename T>
__device__ __forceinline__ T lg_ld(const uint8_t* p)
{
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

__device__ __forceinline__ uint16_t lg_ld16(const uint8_t* p) { return lg_ld<uint16_t>(p); }

__device__ __forceinline__ int lg_dot4(int a, int b, int c)
{
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

/* sum over aligned groups of G lanes (G a power of two <= 64) */
template <int G>
__device__ __forceinline__ float lg_group_sum(float v)
{
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LG_WAVE);
    return v;
}

template <int G>
__device__ __forceinline__ float lg_group_max(float v)
{
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, LG_WAVE));
    return v;
}

template <int G>
__device__ __forceinline__ int lg_group_isum(int v)
{
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LG_WAVE);
    return v;
}

/* block-wide float sum over blockDim.x threads (multiple of 64) via LDS;
 * every thread gets the result.  red must hold blockDim.x/64 floats. */
__device__ __forceinline__ float lg_block_sum(float v, float* red)
{
    v = lg_group_sum<LG_WAVE>(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

/* host helper: turn a failed kernel launch into LG_ERR_HIP */
int lg_check_launch(const char* what);

/* internal launchers (lg_kernels.hip) */
int lg_launch_quantize_q8_0(const float* x, int64_t n, void* y, hipStream_t s);
int lg_launch_quantize_q8_K(const float* x, int64_t n, void* y, hipStream_t s);
int lg_launch_dequantize(int type, const void* x, float* y, int64_t n, hipStream_t s);
int lg_launch_rmsnorm_quant(const float* x, const float* w, int n, float eps, int qtype, void* out_q, float* out_f,
                            hipStream_t s);
int lg_launch_swiglu_quant(float* hb, const float* hb2, int n, int qtype, void* out_q, hipStream_t s);
int lg_launch_qk_norm_rope_kv(float* q, float* k, const float* v, const float* qw, const float* kw, int n_heads,
                              int n_kv_heads, int head_dim, int rope_dim, int pos, const float* freq, float eps,
                              uint16_t* kc_row, uint16_t* vc_row, hipStream_t s);
int lg_launch_embed(int type, const uint8_t* table, uint32_t rsz, const int* tok_dev, int tok, int n, float* x,
                    hipStream_t s);
int lg_launch_argmax(const float* x, int n, int* out, hipStream_t s);

/* lg_matvec.hip */
int lg_launch_matvec(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, int accumulate,
                     hipStream_t s);

/* lg_attn.hip */
size_t lg_attn_ws_bytes(int n_heads, int head_dim, int pos);
int lg_launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* ws, size_t ws_bytes,
                   hipStream_t s);
