/* Top-p / top-k sampling of a device logits vector (sampler_topp,
 * fast/ligguf_fast_qk.cpp:172-214), so that a sampled decode loop needs no
 * logits copy to the host.
 *
 * The reference: p_i = expf((l_i - max) / temp) (inv_temp = 1 / temp,
 * :178-186), normalised by their sum (:189), sorted by p descending, ties by
 * token ascending (qsort with cmp_sampler_ent_desc, :162-170, :190); top =
 * topp, or p of the first entry when topp <= 0, at most 1 (:192-194); the
 * cutoff is the first index whose cumulative p reaches top, at most topk - 1
 * (:195-204); r = rand() / RAND_MAX * cum (:206) selects the first entry
 * whose cumulative p reaches r (:207-213).  temp <= 0 and a sum <= 0 give the
 * greedy token (:176, :188).
 *
 * Here: one pass for the first-index argmax per block, one for p and its
 * block sums, one normalising p by the total, a stable descending radix sort
 * of (p, token) -- equal p keep ascending tokens, the reference's tie rule --
 * and one workgroup scanning the sorted p in tiles of 8192 (8 consecutive
 * entries per thread) until the cutoff, then finding r among the scanned
 * sums.  The host passes the uniform draw
 * rand() / RAND_MAX.  Cumulative sums are tree sums, the reference's are
 * sequential: the sampled token is the reference's except where r or top
 * lies within float rounding of a cumulative sum. */
#include <rocprim/device/device_radix_sort.hpp>
#include "lg_common.h"

#define LG_SMP_T 256                /* threads of the elementwise passes */
#define LG_SMP_PER (LG_SMP_T * 4)   /* logits per block */
#define LG_SMP_MAXB 1024            /* blocks at most (grid-stride past that) */
#define LG_SMP_SCAN 1024            /* threads of the scanning workgroup */
#define LG_SMP_PT 8                 /* consecutive sorted entries per scanning thread and tile */

struct LgSampleWs {
    int n;
    int nb;
    float* p;          /* [n] */
    int* tok;          /* [n] */
    float* ps;         /* [n] sorted descending */
    int* ts;           /* [n] */
    float* cum;        /* [n] cumulative sums of ps, up to the cutoff */
    float* bmax;       /* [LG_SMP_MAXB] */
    int* bidx;         /* [LG_SMP_MAXB] */
    float* bsum;       /* [LG_SMP_MAXB] */
    int* out;          /* [1] */
    void* tmp;
    size_t tmp_bytes;
};

/* (v, i) better than (w, j): larger, or equal and earlier (strict > scan of
 * sampler_greedy, fast/ligguf_fast_qk.cpp:146-160) */
__device__ __forceinline__ bool smp_better(float v, int i, float w, int j)
{
    return v > w || (v == w && i < j);
}

template <int NT>
__device__ __forceinline__ void smp_block_argmax(float& v, int& i)
{
    __shared__ float sv[NT / 64];
    __shared__ int si[NT / 64];
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o);
        const int j = __shfl_xor(i, o);
        if (smp_better(w, j, v, i)) { v = w; i = j; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int k = 1; k < NT / 64; k++)
        if (smp_better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
    __syncthreads();
}

template <int NT>
__device__ __forceinline__ float smp_block_sum(float v)
{
    __shared__ float ss[NT / 64];
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) ss[wave] = v;
    __syncthreads();
    float s = ss[0];
    for (int k = 1; k < NT / 64; k++) s += ss[k];
    __syncthreads();
    return s;
}

/* the global (max, first index) from the block partials, every block the
 * same way */
__device__ __forceinline__ void smp_global_argmax(const LgSampleWs ws, float& v, int& i)
{
    v = -INFINITY;
    i = 0x7fffffff;
    for (int b = threadIdx.x; b < ws.nb; b += LG_SMP_T)
        if (smp_better(ws.bmax[b], ws.bidx[b], v, i)) { v = ws.bmax[b]; i = ws.bidx[b]; }
    smp_block_argmax<LG_SMP_T>(v, i);
}

__device__ __forceinline__ float smp_global_sum(const LgSampleWs ws)
{
    float s = 0.0f;
    for (int b = threadIdx.x; b < ws.nb; b += LG_SMP_T) s += ws.bsum[b];
    return smp_block_sum<LG_SMP_T>(s);
}

__global__ __launch_bounds__(LG_SMP_T) void k_smp_max(const float* __restrict__ x, LgSampleWs ws)
{
    float v = -INFINITY;
    int i = 0x7fffffff;
    for (int j = blockIdx.x * LG_SMP_T + threadIdx.x; j < ws.n; j += gridDim.x * LG_SMP_T)
        if (smp_better(x[j], j, v, i)) { v = x[j]; i = j; }
    smp_block_argmax<LG_SMP_T>(v, i);
    if (threadIdx.x == 0) { ws.bmax[blockIdx.x] = v; ws.bidx[blockIdx.x] = i; }
}

__global__ __launch_bounds__(LG_SMP_T) void k_smp_exp(const float* __restrict__ x, LgSampleWs ws, float inv_temp)
{
    float M;
    int mi;
    smp_global_argmax(ws, M, mi);
    float s = 0.0f;
    for (int j = blockIdx.x * LG_SMP_T + threadIdx.x; j < ws.n; j += gridDim.x * LG_SMP_T) {
        const float p = expf((x[j] - M) * inv_temp);
        ws.p[j] = p;
        ws.tok[j] = j;
        s += p;
    }
    s = smp_block_sum<LG_SMP_T>(s);
    if (threadIdx.x == 0) ws.bsum[blockIdx.x] = s;
}

__global__ __launch_bounds__(LG_SMP_T) void k_smp_norm(LgSampleWs ws)
{
    const float sum = smp_global_sum(ws);
    if (!(sum > 0.0f)) return;   /* the greedy token (k_smp_pick) */
    for (int j = blockIdx.x * LG_SMP_T + threadIdx.x; j < ws.n; j += gridDim.x * LG_SMP_T) ws.p[j] = ws.p[j] / sum;
}

/* exclusive block scan of v (LG_SMP_SCAN threads); returns the block total
 * in *tot */
__device__ __forceinline__ float smp_scan(float v, float* tot)
{
    __shared__ float sw[LG_SMP_SCAN / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int o = 1; o < 64; o <<= 1) {
        const float w = __shfl_up(v, o);
        if (lane >= o) v += w;
    }
    float ex = __shfl_up(v, 1);
    if (lane == 0) ex = 0.0f;
    if (lane == 63) sw[wave] = v;
    __syncthreads();
    float pre = 0.0f, all = 0.0f;
    for (int k = 0; k < LG_SMP_SCAN / 64; k++) {
        if (k < wave) pre += sw[k];
        all += sw[k];
    }
    __syncthreads();
    *tot = all;
    return pre + ex;
}

__device__ __forceinline__ int smp_block_min(int c)
{
    __shared__ int sm[LG_SMP_SCAN / 64];
    for (int o = 32; o > 0; o >>= 1) c = min(c, __shfl_xor(c, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sm[wave] = c;
    __syncthreads();
    int m = sm[0];
    for (int k = 1; k < LG_SMP_SCAN / 64; k++) m = min(m, sm[k]);
    __syncthreads();
    return m;
}

__global__ __launch_bounds__(LG_SMP_SCAN) void k_smp_pick(LgSampleWs ws, float topp, int topk, float r01)
{
    const int tid = threadIdx.x;
    float s = 0.0f;
    for (int b = tid; b < ws.nb; b += LG_SMP_SCAN) s += ws.bsum[b];
    const float sum = smp_block_sum<LG_SMP_SCAN>(s);
    if (!(sum > 0.0f)) {
        float v = -INFINITY;
        int i = 0x7fffffff;
        for (int b = tid; b < ws.nb; b += LG_SMP_SCAN)
            if (smp_better(ws.bmax[b], ws.bidx[b], v, i)) { v = ws.bmax[b]; i = ws.bidx[b]; }
        smp_block_argmax<LG_SMP_SCAN>(v, i);
        if (tid == 0) ws.out[0] = i;
        return;
    }
    float top = topp;
    if (top <= 0.0f) top = ws.ps[0];
    if (top > 1.0f) top = 1.0f;
    const int K = (topk <= 0 || topk > ws.n) ? ws.n : topk;
    /* the cutoff: the first index whose cumulative p reaches top, else K - 1.
     * Tiles of LG_SMP_SCAN * LG_SMP_PT entries, LG_SMP_PT consecutive ones
     * per thread: a running sum in the thread on top of the block's
     * exclusive scan of the thread totals */
    constexpr int TILE = LG_SMP_SCAN * LG_SMP_PT;
    int cutoff = -1;
    float carry = 0.0f;
    for (int base = 0; base < K && cutoff < 0; base += TILE) {
        const int i0 = base + tid * LG_SMP_PT;
        float run[LG_SMP_PT], loc = 0.0f;
#pragma unroll
        for (int k = 0; k < LG_SMP_PT; k++) {
            loc += i0 + k < K ? ws.ps[i0 + k] : 0.0f;
            run[k] = loc;
        }
        float tot;
        const float b = carry + smp_scan(loc, &tot);
        int cand = 0x7fffffff;
#pragma unroll
        for (int k = 0; k < LG_SMP_PT; k++) {
            const float c = b + run[k];
            if (i0 + k < K) {
                ws.cum[i0 + k] = c;
                if (c >= top && cand == 0x7fffffff) cand = i0 + k;
            }
        }
        const int f = smp_block_min(cand);
        if (f != 0x7fffffff) cutoff = f;
        carry += tot;
    }
    if (cutoff < 0) cutoff = K - 1;
    __threadfence_block();
    __syncthreads();
    const float r = r01 * ws.cum[cutoff];
    /* the first entry up to the cutoff whose cumulative p reaches r (each
     * thread reads the sums it wrote, plus the cutoff's) */
    int pick = 0x7fffffff;
    for (int base = 0; base <= cutoff && pick == 0x7fffffff; base += TILE) {
        const int i0 = base + tid * LG_SMP_PT;
        int cand = 0x7fffffff;
#pragma unroll
        for (int k = 0; k < LG_SMP_PT; k++)
            if (i0 + k <= cutoff && cand == 0x7fffffff && ws.cum[i0 + k] >= r) cand = i0 + k;
        pick = smp_block_min(cand);
    }
    if (tid == 0) ws.out[0] = ws.ts[pick == 0x7fffffff ? cutoff : pick];
}

static void smp_free(LgSampleWs* w)
{
    if (!w) return;
    hipFree(w->p);
    hipFree(w->tok);
    hipFree(w->ps);
    hipFree(w->ts);
    hipFree(w->cum);
    hipFree(w->bmax);
    hipFree(w->bidx);
    hipFree(w->bsum);
    hipFree(w->out);
    hipFree(w->tmp);
    delete w;
}

void lg_sample_ws_free(LgSampleWs* w) { smp_free(w); }

int lg_sample_ws_alloc(int n, LgSampleWs** out)
{
    *out = nullptr;
    if (n <= 0) { lg_set_error("sampler: vocabulary size %d", n); return LG_ERR_ARG; }
    LgSampleWs* w = new LgSampleWs();
    w->n = n;
    const int nb = (n + LG_SMP_PER - 1) / LG_SMP_PER;
    w->nb = nb < LG_SMP_MAXB ? nb : LG_SMP_MAXB;
    bool ok = hipMalloc((void**)&w->p, (size_t)n * 4) == hipSuccess && hipMalloc((void**)&w->tok, (size_t)n * 4) == hipSuccess &&
              hipMalloc((void**)&w->ps, (size_t)n * 4) == hipSuccess && hipMalloc((void**)&w->ts, (size_t)n * 4) == hipSuccess &&
              hipMalloc((void**)&w->cum, (size_t)n * 4) == hipSuccess &&
              hipMalloc((void**)&w->bmax, LG_SMP_MAXB * 4) == hipSuccess &&
              hipMalloc((void**)&w->bidx, LG_SMP_MAXB * 4) == hipSuccess &&
              hipMalloc((void**)&w->bsum, LG_SMP_MAXB * 4) == hipSuccess && hipMalloc((void**)&w->out, 16) == hipSuccess;
    if (ok) {
        size_t bytes = 0;
        ok = rocprim::radix_sort_pairs_desc(nullptr, bytes, w->p, w->ps, w->tok, w->ts, (unsigned int)n, 0, 32) == hipSuccess;
        w->tmp_bytes = bytes;
        ok = ok && hipMalloc(&w->tmp, bytes ? bytes : 16) == hipSuccess;
    }
    if (!ok) {
        smp_free(w);
        lg_set_error("sampler: device allocation for %d entries failed", n);
        return LG_ERR_HIP;
    }
    *out = w;
    return LG_OK;
}

int lg_sample_ws_size(const LgSampleWs* w) { return w ? w->n : 0; }

/* token into ws->out (device); temp > 0, 0 <= r01 <= 1 checked by the caller */
int lg_launch_sample_topp(const float* logits, LgSampleWs* w, float temp, float topp, int topk, float r01, hipStream_t s)
{
    const LgSampleWs ws = *w;
    const float inv_temp = 1.0f / temp;
    hipLaunchKernelGGL(k_smp_max, dim3(ws.nb), dim3(LG_SMP_T), 0, s, logits, ws);
    hipLaunchKernelGGL(k_smp_exp, dim3(ws.nb), dim3(LG_SMP_T), 0, s, logits, ws, inv_temp);
    hipLaunchKernelGGL(k_smp_norm, dim3(ws.nb), dim3(LG_SMP_T), 0, s, ws);
    int rc = lg_check_launch("sampler passes");
    if (rc) return rc;
    size_t bytes = ws.tmp_bytes;
    if (rocprim::radix_sort_pairs_desc(ws.tmp, bytes, ws.p, ws.ps, ws.tok, ws.ts, (unsigned int)ws.n, 0, 32, s) !=
        hipSuccess) {
        lg_set_error("sampler: radix sort failed");
        return LG_ERR_HIP;
    }
    hipLaunchKernelGGL(k_smp_pick, dim3(1), dim3(LG_SMP_SCAN), 0, s, ws, topp, topk, r01);
    return lg_check_launch("sampler pick");
}

int* lg_sample_ws_out(LgSampleWs* w) { return w->out; }
