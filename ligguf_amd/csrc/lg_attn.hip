/* lg_attn.hip -- GQA decode attention over the fp16 KV cache for gfx950
 * (the inline attention block of inference(), fast/ligguf_fast_qk.cpp:64-105,
 * with softmax of fast/lil_math.cpp:964-976).
 *
 * Split over the sequence ("flash-decoding"): workgroup (chunk c, KV head
 * kh) takes positions [c*CH, min((c+1)*CH, pos+1)) and all NREP query heads
 * that share kh, so every K/V row is read from HBM once.  A K/V row of one
 * head is HD fp16 = 2*HD bytes; LPP lanes split it (DPL dims each, one
 * 128-bit load when DPL = 8), so a wave covers 64/LPP positions per step.
 *   pass 1: scores s[h][t] = q_h . k_t * scale into LDS (t == pos reads the
 *           fp32 k of this step, as fast/ligguf_fast_qk.cpp:77-79 does);
 *   pass 2: chunk max m and p = exp(s - m), l = sum p;
 *   pass 3: o[h] = sum_t p[h][t] v_t (fp32 v at t == pos, :98-99).
 * The partials (m, l, o) go to the workspace; k_attn_merge rescales them by
 * exp(m_c - M) and divides by the total, which equals the reference's
 * single-pass softmax.
 */
#include <math.h>

#include <mutex>

#include "lg_common.h"

#define LG_ATTN_MAX_CHUNK 1024

/* chunk length for a context of ctx positions: about 128 chunks (with 8 KV
 * heads, 1024 workgroups: four per CU), between 64 and LG_ATTN_MAX_CHUNK
 * positions, multiple of 64 */
static int attn_chunk(int ctx)
{
    int c = (ctx + 127) / 128;
    c = (c + 63) / 64 * 64;
    if (c < 64) c = 64;
    if (c > LG_ATTN_MAX_CHUNK) c = LG_ATTN_MAX_CHUNK;
    return c;
}

size_t lg_attn_ws_bytes(int n_heads, int head_dim, int pos)
{
    if (n_heads <= 0 || head_dim <= 0 || pos < 0) return 0;
    const int ctx = pos + 1;
    const int ch = attn_chunk(ctx);
    const int nch = (ctx + ch - 1) / ch;
    return (size_t)n_heads * nch * (head_dim + 2) * sizeof(float);
}

template <int DPL>
__device__ __forceinline__ void load_half_row(const uint16_t* __restrict__ p, float out[DPL])
{
    if constexpr (DPL == 8) {
        const uint4 v = lg_ld<uint4>((const uint8_t*)p);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[2 * i] = lg_h2f((uint16_t)(u[i] & 0xffffu));
            out[2 * i + 1] = lg_h2f((uint16_t)(u[i] >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < DPL; i++) out[i] = lg_h2f(p[i]);
    }
}

template <int DPL>
__device__ __forceinline__ void load_f32_row(const float* __restrict__ p, float out[DPL])
{
#pragma unroll
    for (int i = 0; i < DPL; i++) out[i] = p[i];
}

/* workspace layout per (kv head kh, chunk c): NREP m, NREP l, NREP*HD o;
 * i.e. per query head h = kh*NREP + r: index ((kh*nch + c)*NREP + r) */
template <int HD, int NREP, int LPP>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ q, const float* __restrict__ kcur,
                                                    const float* __restrict__ vcur, const uint16_t* __restrict__ kc,
                                                    const uint16_t* __restrict__ vc, int kv_dim, int pos, int chunk,
                                                    int nch, float scale, float* __restrict__ ws)
{
    constexpr int DPL = HD / LPP;
    constexpr int PPW = 64 / LPP;      /* positions per wave step */
    constexpr int PPB = 4 * PPW;       /* positions per workgroup step */
    __shared__ float s_sc[NREP * LG_ATTN_MAX_CHUNK];
    __shared__ float s_red[4 * NREP * HD];
    __shared__ float s_m[4 * NREP];

    const int c = blockIdx.x, kh = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane & (LPP - 1), grp = lane / LPP;
    const int t0 = c * chunk;
    int t1 = t0 + chunk;
    if (t1 > pos + 1) t1 = pos + 1;
    const int nt = t1 - t0;

    float qr[NREP][DPL];
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) qr[r][i] = q[(size_t)(kh * NREP + r) * HD + gl * DPL + i];

    /* pass 1: scores, U steps of rows loaded before any is used (positions
     * past the chunk load its first row and are not stored) */
    constexpr int U = 4;
    for (int tb = 0; tb < nt; tb += U * PPB) {
        float kv[U][DPL];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            const int t = tl < nt ? t0 + tl : t0;
            if (t == pos) load_f32_row<DPL>(kcur + kh * HD + gl * DPL, kv[u]);
            else load_half_row<DPL>(kc + (size_t)t * kv_dim + kh * HD + gl * DPL, kv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
#pragma unroll
            for (int r = 0; r < NREP; r++) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < DPL; i++) s += qr[r][i] * kv[u][i];
                s = lg_group_sum<LPP>(s);
                if (gl == 0 && tl < nt) s_sc[r * LG_ATTN_MAX_CHUNK + tl] = s * scale;
            }
        }
    }
    __syncthreads();

    /* pass 2: chunk max and exponentials (each wave scans for all heads) */
    float m[NREP], l[NREP];
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        float mx = -INFINITY;
        for (int i = threadIdx.x; i < nt; i += 256) mx = fmaxf(mx, s_sc[r * LG_ATTN_MAX_CHUNK + i]);
        mx = lg_group_max<64>(mx);
        if (lane == 0) s_m[wave * NREP + r] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        m[r] = fmaxf(fmaxf(s_m[r], s_m[NREP + r]), fmaxf(s_m[2 * NREP + r], s_m[3 * NREP + r]));
        float sum = 0.0f;
        for (int i = threadIdx.x; i < nt; i += 256) {
            const float p = expf(s_sc[r * LG_ATTN_MAX_CHUNK + i] - m[r]);
            s_sc[r * LG_ATTN_MAX_CHUNK + i] = p;
            sum += p;
        }
        l[r] = sum;   /* partial; reduced below */
    }
    __syncthreads();

    /* pass 3: p . V */
    float o[NREP][DPL];
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) o[r][i] = 0.0f;
    for (int tb = 0; tb < nt; tb += U * PPB) {
        float vv[U][DPL];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            const int t = tl < nt ? t0 + tl : t0;
            if (t == pos) load_f32_row<DPL>(vcur + kh * HD + gl * DPL, vv[u]);
            else load_half_row<DPL>(vc + (size_t)t * kv_dim + kh * HD + gl * DPL, vv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            if (tl < nt) {
#pragma unroll
                for (int r = 0; r < NREP; r++) {
                    const float p = s_sc[r * LG_ATTN_MAX_CHUNK + tl];
#pragma unroll
                    for (int i = 0; i < DPL; i++) o[r][i] += p * vv[u][i];
                }
            }
        }
    }
    /* reduce o over the position groups of the wave, then over waves */
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) {
            float v = o[r][i];
#pragma unroll
            for (int off = LPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
            o[r][i] = v;
        }
    if (grp == 0) {
#pragma unroll
        for (int r = 0; r < NREP; r++)
#pragma unroll
            for (int i = 0; i < DPL; i++) s_red[(wave * NREP + r) * HD + gl * DPL + i] = o[r][i];
    }
    /* l: block sum per head */
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        float v = lg_group_sum<64>(l[r]);
        l[r] = v;
    }
    __syncthreads();
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NREP; r++) s_m[wave * NREP + r] = l[r];
    }
    __syncthreads();
    float* out = ws + ((size_t)kh * nch + c) * NREP * (HD + 2);
    for (int i = threadIdx.x; i < NREP * HD; i += 256) {
        const int r = i / HD, dd = i % HD;
        out[2 * NREP + r * HD + dd] = s_red[(0 * NREP + r) * HD + dd] + s_red[(1 * NREP + r) * HD + dd] +
                                      s_red[(2 * NREP + r) * HD + dd] + s_red[(3 * NREP + r) * HD + dd];
    }
    if (threadIdx.x < NREP) {
        const int r = threadIdx.x;
        out[r] = m[r];
        out[NREP + r] = s_m[r] + s_m[NREP + r] + s_m[2 * NREP + r] + s_m[3 * NREP + r];
    }
}

/* one workgroup per query head: merge the chunk partials */
template <int HD, int NREP>
__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ ws, int nch, float* __restrict__ out)
{
    const int h = blockIdx.x;
    const int kh = h / NREP, r = h % NREP;
    float M = -INFINITY;
#pragma unroll 8
    for (int c = 0; c < nch; c++) M = fmaxf(M, ws[((size_t)kh * nch + c) * NREP * (HD + 2) + r]);
    for (int dd = threadIdx.x; dd < HD; dd += blockDim.x) {
        float L = 0.0f, acc = 0.0f;
#pragma unroll 8
        for (int c = 0; c < nch; c++) {
            const float* p = ws + ((size_t)kh * nch + c) * NREP * (HD + 2);
            const float w = expf(p[r] - M);
            L += p[NREP + r] * w;
            acc += p[2 * NREP + r * HD + dd] * w;
        }
        out[(size_t)h * HD + dd] = acc / L;
    }
}

template <int HD, int NREP, int LPP>
static void launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                        int n_kv_heads, int pos, float* out, float* ws, hipStream_t s)
{
    const int ctx = pos + 1;
    const int ch = attn_chunk(ctx);
    const int nch = (ctx + ch - 1) / ch;
    const float scale = 1.0f / sqrtf((float)HD);
    hipLaunchKernelGGL((k_attn_split<HD, NREP, LPP>), dim3(nch, n_kv_heads), dim3(256), 0, s, q, k, v, kc, vc,
                       n_kv_heads * HD, pos, ch, nch, scale, ws);
    hipLaunchKernelGGL((k_attn_merge<HD, NREP>), dim3(n_kv_heads * NREP), dim3(HD < 256 ? (HD + 63) / 64 * 64 : 256), 0, s,
                       ws, nch, out);
}

template <int HD, int LPP>
static int attn_nrep(int nrep, const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                     int n_kv_heads, int pos, float* out, float* ws, hipStream_t s)
{
    switch (nrep) {
    case 1: launch_attn<HD, 1, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 2: launch_attn<HD, 2, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 4: launch_attn<HD, 4, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 8: launch_attn<HD, 8, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    default: lg_set_error("attention: %d query heads per KV head unsupported (1, 2, 4, 8)", nrep); return LG_ERR_ARG;
    }
}

int lg_launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* ws, size_t ws_bytes,
                   hipStream_t s)
{
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || pos < 0 || !q || !k || !v || !out || !ws ||
        (pos > 0 && (!kc || !vc))) {
        lg_set_error("attention: bad arguments (heads %d/%d, pos %d)", n_heads, n_kv_heads, pos);
        return LG_ERR_ARG;
    }
    if (ws_bytes < lg_attn_ws_bytes(n_heads, head_dim, pos)) {
        lg_set_error("attention: workspace of %zu bytes, %zu needed", ws_bytes, lg_attn_ws_bytes(n_heads, head_dim, pos));
        return LG_ERR_ARG;
    }
    const int nrep = n_heads / n_kv_heads;
    float* w = (float*)ws;
    int rc;
    switch (head_dim) {
    case 48: rc = attn_nrep<48, 8>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 64: rc = attn_nrep<64, 8>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 128: rc = attn_nrep<128, 16>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 256: rc = attn_nrep<256, 32>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    default: lg_set_error("attention: head_dim %d unsupported (48, 64, 128, 256)", head_dim); return LG_ERR_ARG;
    }
    if (rc) return rc;
    return lg_check_launch("attention");
}

/* ------------------------------------------------------------------ */
/* lg_attn_decode_noalloc: the same kernels on a scratch area that the */
/* library holds in device memory for the life of the process          */
/* ------------------------------------------------------------------ */
/* 8 MiB per device: lg_attn_ws_bytes for 32 heads of 128 at up to
 * 131072 positions (128 chunks of 1024), or 64 heads of 128 at up to
 * 65536.  Every partial is written before it is read, so nothing needs
 * clearing between calls. */
#define LG_ATTN_SCRATCH_BYTES ((size_t)8 << 20)
#define LG_ATTN_SCRATCH_DEVICES 64

static __device__ __align__(256) float scratch[LG_ATTN_SCRATCH_BYTES / sizeof(float)];

/* the device address of `scratch` on each device, looked up once per device
 * (with that device current) at the entry point's first call there; host code
 * passes only these addresses to kernels */
static void* g_scratch_dev[LG_ATTN_SCRATCH_DEVICES];
static std::mutex g_scratch_mu;

static int attn_scratch(void** out)
{
    int dev = 0;
    LG_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= LG_ATTN_SCRATCH_DEVICES) {
        lg_set_error("attention scratch: device %d beyond the %d supported", dev, LG_ATTN_SCRATCH_DEVICES);
        return LG_ERR_ARG;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            lg_set_error("attention scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
            return LG_ERR_HIP;
        }
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return LG_OK;
}

extern "C" size_t lg_attn_scratch_bytes(void) { return LG_ATTN_SCRATCH_BYTES; }

extern "C" int lg_attn_decode_noalloc(const float* q, const float* k, const float* v, const uint16_t* kc,
                                      const uint16_t* vc, int n_heads, int n_kv_heads, int head_dim, int pos,
                                      float* out, void* stream)
{
    const size_t need = lg_attn_ws_bytes(n_heads, head_dim, pos);
    if (need > LG_ATTN_SCRATCH_BYTES) {
        lg_set_error("attention (no allocation): %zu bytes of partials needed for %d heads of %d at position %d, "
                     "the scratch area holds %zu", need, n_heads, head_dim, pos, LG_ATTN_SCRATCH_BYTES);
        return LG_ERR_ARG;
    }
    void* ws = nullptr;
    const int rc = attn_scratch(&ws);
    if (rc) return rc;
    return lg_launch_attn(q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos, out, ws, LG_ATTN_SCRATCH_BYTES,
                          (hipStream_t)stream);
}
