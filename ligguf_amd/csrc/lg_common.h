/* lg_common.h -- shared device helpers of the gfx950 decode path. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/ligguf_hip.h"

/* GGUF block byte sizes and field offsets (fast/lil_gguf.h:64-119) */
#define LG_QK8_0 32
#define LG_QK_K 256
/* internal forms of Q8_0 / Q6_K rows regrouped for aligned loads (copies the
 * whole-step kernels read; Fmt<LG_Q8_0_R> in lg_fmt.h) */
#define LG_Q8_0_R 108
#define LG_Q6_K_R 114
#define LG_Q1_G_R 141
#define LG_Q3_K_R 111
#define LG_Q1_0_R 140
/* internal forms of F16 / F32 rows in the whole-step kernels: the fp32
 * activation they multiply stays in LDS (Fmt<LG_F16_L>, Fmt<LG_F32_L> in
 * lg_phase.h) */
#define LG_F16_L 101
#define LG_F32_L 102
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

/* Cross-lane butterfly.  Step K pairs every lane with a partner so that
 * after steps 0..log2(G)-1 each aligned group of G lanes has combined all of
 * its members: steps 0-3 are DPP permutes inside 16-lane rows (quad_perm
 * [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror -- each pairs
 * two already-combined halves), steps 4-5 cross rows (v_permlane16_swap,
 * v_permlane32_swap: VALU, no LDS round trip).  Every
 * lane ends with the same bits: each pairwise op sees the same two operands. */
#define LG_DPP_XOR1 0xB1
#define LG_DPP_XOR2 0x4E
#define LG_DPP_HALF_MIRROR 0x141
#define LG_DPP_MIRROR 0x140

/* every lane of these permutes reads a valid lane of its row, so bound_ctrl
 * changes nothing; with it the compiler folds the move into the consuming
 * add/max (v_add_f32_dpp ...) */
template <int CTRL>
__device__ __forceinline__ int lg_dpp(int v)
{
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

template <int K>
__device__ __forceinline__ int lg_partner(int v)
{
    if constexpr (K == 0) return lg_dpp<LG_DPP_XOR1>(v);
    else if constexpr (K == 1) return lg_dpp<LG_DPP_XOR2>(v);
    else if constexpr (K == 2) return lg_dpp<LG_DPP_HALF_MIRROR>(v);
    else if constexpr (K == 3) return lg_dpp<LG_DPP_MIRROR>(v);
    else if constexpr (K == 4) {
        /* lane ^ 16: v_permlane16_swap gives even rows the row above ([1])
         * and odd rows the row below ([0]) */
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((__lane_id() & 16) ? r[0] : r[1]);
    } else {
        /* lane ^ 32: v_permlane32_swap, lanes 0..31 get [1], 32..63 [0] */
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((__lane_id() & 32) ? r[0] : r[1]);
    }
}

template <int K>
__device__ __forceinline__ float lg_partner(float v)
{
    return __int_as_float(lg_partner<K>(__float_as_int(v)));
}

/* a*b + c*d rounded one fixed way, fma(c, d, a*b): in an expression of two
 * products the compiler picks which product it fuses into the add, and may
 * pick differently in different kernels -- the paths would then disagree in
 * the last bit */
__device__ __forceinline__ float lg_fma2(float a, float b, float c, float d)
{
    return __builtin_fmaf(c, d, a * b);
}

/* x^2 + y^2 + z^2 + w^2 in one fixed order */
__device__ __forceinline__ float lg_sq4(float4 t)
{
    return __builtin_fmaf(t.w, t.w, __builtin_fmaf(t.z, t.z, __builtin_fmaf(t.y, t.y, t.x * t.x)));
}

/* sum over aligned groups of G lanes (G a power of two <= 64) */
template <int G>
__device__ __forceinline__ float lg_group_sum(float v)
{
    if constexpr (G >= 2) v += lg_partner<0>(v);
    if constexpr (G >= 4) v += lg_partner<1>(v);
    if constexpr (G >= 8) v += lg_partner<2>(v);
    if constexpr (G >= 16) v += lg_partner<3>(v);
    if constexpr (G >= 32) v += lg_partner<4>(v);
    if constexpr (G >= 64) v += lg_partner<5>(v);
    return v;
}

/* sum over the 64 lanes of a wave, returned as a wave-uniform value: the
 * 16-lane rows by the butterfly, then DPP row_bcast:15 / row_bcast:31 carry
 * the row sums up to lane 63 ((r3 + r2) + (r1 + r0)), read back as a scalar
 * -- no cross-row permute through LDS */
#define LG_DPP_ROW_BCAST15 0x142
#define LG_DPP_ROW_BCAST31 0x143
__device__ __forceinline__ float lg_wave_sum(float v)
{
    v = lg_group_sum<16>(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), LG_DPP_ROW_BCAST15, 0xA, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), LG_DPP_ROW_BCAST31, 0xC, 0xF, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* sum of x[0..n)^2 by one wave (n a multiple of 256), in the order of the
 * whole-step kernels' rmsnorm build: the 256-value chunks in 8 interleaved
 * groups (chunk % 8), lane partials in chunk order, one lg_wave_sum per
 * group, the group sums added in group order */
__device__ __forceinline__ float lg_sumsq_chunked(const float* __restrict__ x, int n, int lane)
{
    float ss = 0.0f;
    for (int w = 0; w < 8; w++) {
        float p = 0.0f;
        for (int i = 256 * w + 4 * lane; i < n; i += 2048) p += lg_sq4(*(const float4*)(x + i));
        ss += lg_wave_sum(p);
    }
    return ss;
}

/* the value of the 16-lane row above (row r+1 for even r; odd rows get their
 * own) and of the lane 32 above (lanes 0..31): v_permlane16_swap /
 * v_permlane32_swap, VALU with no LDS round trip */
__device__ __forceinline__ float lg_from_row_above(float x)
{
    return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}

__device__ __forceinline__ float lg_from_half_above(float x)
{
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}

template <int G>
__device__ __forceinline__ float lg_group_max(float v)
{
    if constexpr (G >= 2) v = fmaxf(v, lg_partner<0>(v));
    if constexpr (G >= 4) v = fmaxf(v, lg_partner<1>(v));
    if constexpr (G >= 8) v = fmaxf(v, lg_partner<2>(v));
    if constexpr (G >= 16) v = fmaxf(v, lg_partner<3>(v));
    if constexpr (G >= 32) v = fmaxf(v, lg_partner<4>(v));
    if constexpr (G >= 64) v = fmaxf(v, lg_partner<5>(v));
    return v;
}

/* max over aligned groups of G lanes of non-negative floats (|x| values),
 * taken on their bits as unsigned integers -- the same order for
 * non-negative floats; an integer max folds into the DPP move and needs no
 * NaN canonicalization */
template <int G>
__device__ __forceinline__ float lg_group_max_nn(float v)
{
    uint32_t u = __float_as_uint(v);
    if constexpr (G >= 2) u = max(u, (uint32_t)lg_partner<0>((int)u));
    if constexpr (G >= 4) u = max(u, (uint32_t)lg_partner<1>((int)u));
    if constexpr (G >= 8) u = max(u, (uint32_t)lg_partner<2>((int)u));
    if constexpr (G >= 16) u = max(u, (uint32_t)lg_partner<3>((int)u));
    if constexpr (G >= 32) u = max(u, (uint32_t)lg_partner<4>((int)u));
    if constexpr (G >= 64) u = max(u, (uint32_t)lg_partner<5>((int)u));
    return __uint_as_float(u);
}

/* wave max of non-negative floats, wave-uniform: the row maxima, then
 * row_bcast:15 / row_bcast:31 up to lane 63 (as lg_wave_sum) */
__device__ __forceinline__ float lg_wave_max_nn(float v)
{
    uint32_t u = __float_as_uint(lg_group_max_nn<16>(v));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, LG_DPP_ROW_BCAST15, 0xA, 0xF, false));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, LG_DPP_ROW_BCAST31, 0xC, 0xF, false));
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)u, 63));
}

template <int G>
__device__ __forceinline__ int lg_group_isum(int v)
{
    if constexpr (G >= 2) v += lg_partner<0>(v);
    if constexpr (G >= 4) v += lg_partner<1>(v);
    if constexpr (G >= 8) v += lg_partner<2>(v);
    if constexpr (G >= 16) v += lg_partner<3>(v);
    if constexpr (G >= 32) v += lg_partner<4>(v);
    if constexpr (G >= 64) v += lg_partner<5>(v);
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

/* The HIP runtime's device initialisation draws numbers from the C library's
 * rand(), which shifts a caller's seeded sequence -- the reference samples
 * top-p with rand() after srand(seed) (fast/ligguf_fast_qk.cpp:204,487-489),
 * so its output would change with the library linked in.  Calls that may
 * initialise the runtime run with a private generator state swapped in
 * (initstate/setstate leave the caller's state untouched meanwhile); another
 * thread calling rand() during lg_create would draw from the private state. */
struct lg_rand_guard {
    char buf[256];
    char* caller;
    lg_rand_guard() { caller = initstate(1u, buf, sizeof(buf)); }
    ~lg_rand_guard() { setstate(caller); }
};

/* host helper: turn a failed kernel launch into LG_ERR_HIP */
int lg_check_launch(const char* what);
int lg_launch_read_probe(const void* buf, size_t bytes, hipStream_t s);

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

/* lg_sample.hip: top-p / top-k sampling on the device */
struct LgSampleWs;
int lg_sample_ws_alloc(int n, LgSampleWs** out);
void lg_sample_ws_free(LgSampleWs* w);
int lg_sample_ws_size(const LgSampleWs* w);
int* lg_sample_ws_out(LgSampleWs* w);
int* lg_sample_ws_out_host(LgSampleWs* w);   /* pinned host word the top-p launches also write */
int lg_launch_sample_topp(const float* logits, LgSampleWs* w, float temp, float topp, int topk, float r01,
                          hipStream_t s);

/* lg_matvec.hip */
int lg_launch_matvec(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, int accumulate,
                     hipStream_t s);

/* lg_attn.hip */
size_t lg_attn_ws_bytes(int n_heads, int head_dim, int pos);
/* looks up the no-allocation attention's scratch address on the current device */
int lg_attn_scratch_setup(void);
int lg_launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* ws, size_t ws_bytes,
                   hipStream_t s);
