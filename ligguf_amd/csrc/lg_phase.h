/* lg_phase.h -- the phases of the per-token step as device code shared by
 * the persistent kernel (lg_persist.hip: one launch walks all phases with
 * flag syncs) and the fused per-phase kernels (lg_fused.hip: one kernel per
 * phase, kernel boundaries as the syncs).  A phase with wait_target == 0 and
 * sig == 0 runs without flag syncs.
 */
#pragma once

#include <math.h>

#include "lg_common.h"
#include "lg_fmt.h"
#include "lg_quant.h"
#include "lg_persist.h"

#define PK_WAVES (PK_THREADS / 64)

/* ------------------------------------------------------------------ */
/* LDS                                                                  */
/* ------------------------------------------------------------------ */
/* activation build area: fp32 staging of x (rmsnorm) + quantized blocks */
__shared__ __attribute__((aligned(16))) float s_x[PK_MAX_EMBED];
__shared__ __attribute__((aligned(16))) uint8_t s_act[(PK_MAX_FF / 256) * LG_BS_Q8_K + 64];
__shared__ float s_red[64];
__shared__ int s_int[8];
/* attention */
__shared__ __attribute__((aligned(16))) float s_q[PK_MAX_NREP * 128];
__shared__ __attribute__((aligned(16))) float s_kv[2 * 128];
__shared__ __attribute__((aligned(16))) float s_sc[PK_MAX_NREP * PK_MAX_CHUNK];
__shared__ __attribute__((aligned(16))) float s_o[PK_WAVES * PK_MAX_NREP * 128];
__shared__ float s_m[PK_WAVES * PK_MAX_NREP];

/* ------------------------------------------------------------------ */
/* coherent memory helpers                                              */
/* ------------------------------------------------------------------ */
template <typename T>
__device__ __forceinline__ T cld(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ void cst(T* p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* two consecutive floats (8-byte aligned) in one coherent load */
__device__ __forceinline__ float2 cld2(const float* p)
{
    const uint64_t u = cld((const uint64_t*)p);
    return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}

/* workgroup barrier that orders LDS but leaves global loads in flight */
__device__ __forceinline__ void bar()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void wait_stores()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

/* publish: every wave's stores acknowledged, then the WG's progress word */
__device__ __forceinline__ void pk_signal(const PkParams& P, uint64_t val)
{
    wait_stores();
    bar();
    if (threadIdx.x == 0) cst(&P.progress[blockIdx.x], val);
}

/* wait until every WG's progress word reaches `target` (wave 0 polls) */
__device__ __forceinline__ void pk_wait(const PkParams& P, uint64_t target)
{
    if (threadIdx.x < 64) {
        if (!cld(P.err)) {
            const int nwg = gridDim.x;
            bool ok = false;
            int it = 0;
            do {
                uint64_t mn = ~0ull;
                for (int i = threadIdx.x; i < nwg; i += 64) {
                    const uint64_t v = cld(&P.progress[i]);
                    mn = v < mn ? v : mn;
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const uint64_t t = __shfl_xor(mn, o, 64);
                    mn = t < mn ? t : mn;
                }
                ok = mn >= target;
            } while (!ok && ++it < P.spin_cap);
            if (!ok && threadIdx.x == 0) cst(P.err, 1u);
        }
    }
    bar();
}

/* phase timestamps (lane 0 of wave 0 of every WG; nothing when tr is NULL) */
__device__ __forceinline__ void stamp(uint64_t* tr, int k)
{
    if (tr && threadIdx.x == 0) tr[k] = wall_clock64();
}

/* ------------------------------------------------------------------ */
/* activation builders (all PK_THREADS threads; end with a barrier)     */
/* ------------------------------------------------------------------ */
/* The activation of width n = CPW * 256 * PK_WAVES is handled as 256-value
 * chunks, chunk (wave + PK_WAVES*c) by wave `wave`, lane l holding values
 * 4l..4l+3 of it.  Every global load of a build is issued before the first
 * one is used, so a build costs one memory round trip.  Activations are
 * read with plain (L2-cached) loads: every activation buffer of a launch is
 * written exactly once, before anyone reads it, so no L2 holds a stale copy
 * (the launch starts with invalidated caches). */
enum { BLD_RMS = 0, BLD_PLAIN = 1 };

__device__ __forceinline__ int chunk_base(int c)
{
    return ((threadIdx.x >> 6) + PK_WAVES * c) * 256 + 4 * (threadIdx.x & 63);
}

/* rmsnorm weights of this wave's chunks: constants, loaded before the wait */
template <int CPW>
struct NormW {
    float4 g[CPW];
    __device__ __forceinline__ void load(const float* __restrict__ w)
    {
#pragma unroll
        for (int c = 0; c < CPW; c++) g[c] = *(const float4*)(w + chunk_base(c));
    }
};

/* this wave's chunks of an activation source vector, loaded on their own
 * so that they can be issued ahead of the weight loads (a wave's loads
 * return in issue order) */
template <int CPW>
struct ActSrc {
    float4 v[CPW];
    __device__ __forceinline__ void load(const float* __restrict__ src)
    {
#pragma unroll
        for (int c = 0; c < CPW; c++) v[c] = *(const float4*)(src + chunk_base(c));
    }
};

/* rmsnorm(x) * w quantized into s_act (fast/lil_math.cpp:922-929 and
 * quantize_q8_K / quantize_q8_0, :329-394).  The sum of squares is taken by
 * one wave in the per-lane order of k_rmsnorm_quant, so both paths agree bit
 * for bit.  x is `src` or, for layer 0 (src == NULL), the embedding row of
 * tok, dequantized here; WG 0 also stores that row as the residual stream
 * `emb_out`. */
template <int QT, int CPW>
__device__ __forceinline__ void build_rms(const PkParams& P, int tok, const NormW<CPW>& nw, const ActSrc<CPW>& xsrc,
                                          bool from_embed, float* __restrict__ emb_out)
{
    constexpr int n = CPW * 256 * PK_WAVES;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float4 xv[CPW];
    if (from_embed) {
        /* one dequantization loop (the switch over types stays out of the
         * unrolled chunk code), staged through s_x */
        const uint8_t* row = P.embd + (size_t)tok * P.embd_rsz;
        for (int i = threadIdx.x; i < n; i += PK_THREADS) s_x[i] = lg_dq_value(P.embd_t, row, i);
        bar();
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            const int b = chunk_base(c);
            xv[c] = *(const float4*)(s_x + b);
            if (blockIdx.x == 0) {
                cst(&emb_out[b], xv[c].x); cst(&emb_out[b + 1], xv[c].y);
                cst(&emb_out[b + 2], xv[c].z); cst(&emb_out[b + 3], xv[c].w);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            xv[c] = xsrc.v[c];
            *(float4*)(s_x + chunk_base(c)) = xv[c];
        }
    }
    bar();
    if (wave == 0) {
        float ss = 0.0f;
        for (int i = 4 * lane; i < n; i += 256) {
            const float4 t = *(const float4*)(s_x + i);
            ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
        }
        ss = lg_group_sum<64>(ss);
        if (lane == 0) s_red[0] = 1.0f / sqrtf(ss / (float)n + P.eps);
    }
    bar();
    const float scale = s_red[0];
#pragma unroll
    for (int c = 0; c < CPW; c++) {
        const float4 t = xv[c], g = nw.g[c];
        const float v[4] = {t.x * scale * g.x, t.y * scale * g.y, t.z * scale * g.z, t.w * scale * g.w};
        lg_emit(v, QT, s_act, wave + PK_WAVES * c, 256);
    }
    bar();
}

/* the source chunks quantized into s_act */
template <int QT, int CPW>
__device__ __forceinline__ void build_plain(const ActSrc<CPW>& a)
{
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < CPW; c++) {
        const float v[4] = {a.v[c].x, a.v[c].y, a.v[c].z, a.v[c].w};
        lg_emit(v, QT, s_act, wave + PK_WAVES * c, 256);
    }
    bar();
}

/* ------------------------------------------------------------------ */
/* matvec phases                                                        */
/* ------------------------------------------------------------------ */
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

/* Items of one phase are split evenly over all waves of the grid in
 * contiguous runs; an item is K rows (K = 2 for up|gate: rows i and i+kstride)
 * each dotted by the whole wave (lane j owns slots j, j+64, ...). */
template <int FMT, int NS, int MAXB, int K>
struct Rows {
    typename Fmt<FMT>::W w[MAXB][K][NS];

    __device__ __forceinline__ void load(const uint8_t* __restrict__ W, uint32_t rsz, int i0, int nb, int kstride,
                                         int lane)
    {
#pragma unroll
        for (int b = 0; b < MAXB; b++) {
            if (b < nb) {
#pragma unroll
                for (int k = 0; k < K; k++) {
                    const uint8_t* row = W + (size_t)(i0 + b + k * kstride) * rsz;
#pragma unroll
                    for (int s = 0; s < NS; s++) Fmt<FMT>::load_w(w[b][k][s], row, lane + 64 * s);
                }
            }
        }
    }
};

/* One matvec phase.  Before the dependency wait, waves 1.. issue the loads
 * of their first MAXB items, the rmsnorm weights and (EPI_RESID) the
 * residual values of their rows -- `res` is stable from phase entry on, the
 * phase that wrote it being two syncs back.  Wave 0 polls the progress
 * words; its own loads go after the wait, since a wave's loads return in
 * order and would hold the poll back.  Then: build the activation, compute,
 * store, publish.  CPW = 256-value activation chunks per wave; DB =
 * double-buffer the items (long phases: the output head). */
template <int FMT, int NS, int MAXB, int K, int EPI, int BLD, int CPW, bool DB>
__device__ __forceinline__ void phase_mv(const PkParams& P, int tok, const uint8_t* __restrict__ W, uint32_t rsz,
                                         int items, int kstride, const float* __restrict__ normw,
                                         const float* __restrict__ src, const float* __restrict__ res_src,
                                         float* __restrict__ out, float* __restrict__ emb_out,
                                         uint64_t wait_target, uint64_t sig, uint64_t* tr)
{
    using F = Fmt<FMT>;
    constexpr int QT = (FMT == LG_Q8_0 || FMT == LG_Q1_0 || FMT == LG_Q1_G) ? LG_Q8_0 : LG_Q8_K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nwv = gridDim.x * PK_WAVES;
    const int gw = blockIdx.x * PK_WAVES + wave;
    const int ipw = (items + nwv - 1) / nwv;
    const int i0 = gw * ipw;
    const int my = max(0, min(items, i0 + ipw) - i0);

    stamp(tr, 0);
    Rows<FMT, NS, MAXB, K> R0;
    NormW<CPW> nw;
    ActSrc<CPW> as;
    float res[MAXB];
    const bool from_embed = BLD == BLD_RMS && !src;
    const int first = DB ? 1 : MAXB;
    auto prefetch = [&]() {
        R0.load(W, rsz, i0, min(my, first), kstride, lane);
        if (EPI == EPI_RESID) {
#pragma unroll
            for (int b = 0; b < MAXB; b++) res[b] = b < min(my, first) ? res_src[i0 + b] : 0.0f;
        }
    };
    if (!wait_target) {
        /* no dependency wait (fused kernels): the activation and the norm
         * weights go first, the rows after them */
        if (!from_embed) as.load(src);
        if (BLD == BLD_RMS) nw.load(normw);
        prefetch();
    } else {
        if (BLD == BLD_RMS) nw.load(normw);
        if (wave != 0) prefetch();
        pk_wait(P, wait_target);
        if (!from_embed) as.load(src);
        if (wave == 0) prefetch();
    }
    stamp(tr, 1);
    if (BLD == BLD_RMS) build_rms<QT, CPW>(P, tok, nw, as, from_embed, emb_out);
    else build_plain<QT, CPW>(as);
    stamp(tr, 2);

    typename F::Act act[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) F::load_act(act[s], s_act, lane + 64 * s);

    float best = -INFINITY;
    int besti = 0x7fffffff;
    auto process = [&](const Rows<FMT, NS, MAXB, K>& R, const float* rs, int b0, int nb) {
#pragma unroll
        for (int b = 0; b < MAXB; b++) {
            if (b < nb) {
                float acc[K];
#pragma unroll
                for (int k = 0; k < K; k++) {
                    float a = 0.0f;
#pragma unroll
                    for (int s = 0; s < NS; s++) a += F::dot(R.w[b][k][s], act[s], lane + 64 * s);
                    acc[k] = lg_group_sum<64>(a);
                }
                const int i = i0 + b0 + b;
                if (EPI == EPI_LOGITS) {
                    if (acc[0] > best) { best = acc[0]; besti = i; }
                }
                if (lane == 0) {
                    if (EPI == EPI_STORE) cst(&out[i], acc[0]);
                    else if (EPI == EPI_RESID) cst(&out[i], rs[b] + acc[0]);
                    else if (EPI == EPI_SWIGLU) {
                        const float u = acc[0], g = acc[1];
                        cst(&out[i], (g / (1.0f + expf(-g))) * u);
                    } else out[i] = acc[0];
                }
            }
        }
    };
    if (!DB) {
        for (int b0 = 0; b0 < my; b0 += MAXB) {
            const int nb = min(MAXB, my - b0);
            if (b0 > 0) {
                R0.load(W, rsz, i0 + b0, nb, kstride, lane);
                if (EPI == EPI_RESID) {
#pragma unroll
                    for (int b = 0; b < MAXB; b++) res[b] = b < nb ? res_src[i0 + b0 + b] : 0.0f;
                }
            }
            process(R0, res, b0, nb);
        }
    } else {
        /* R0 holds the first FIRST items (issued before the build, so the
         * activation loads are not queued behind a flood of rows); then
         * two batches in flight: the next loads while this one computes */
        Rows<FMT, NS, MAXB, K> R1;
        float res1[MAXB];
        auto load_res = [&](float* r, int b0, int nb) {
            if (EPI == EPI_RESID) {
#pragma unroll
                for (int b = 0; b < MAXB; b++) r[b] = b < nb ? res_src[i0 + b0 + b] : 0.0f;
            }
        };
        int c0 = 0, n0 = min(my, first);
        while (n0 > 0) {
            const int c1 = c0 + n0;
            const int n1 = min(MAXB, my - c1);
            if (n1 > 0) {
                R1.load(W, rsz, i0 + c1, n1, kstride, lane);
                load_res(res1, c1, n1);
            }
            process(R0, res, c0, n0);
            const int c2 = c1 + max(n1, 0);
            const int n2 = n1 > 0 ? min(MAXB, my - c2) : 0;
            if (n2 > 0) {
                R0.load(W, rsz, i0 + c2, n2, kstride, lane);
                load_res(res, c2, n2);
            }
            if (n1 > 0) process(R1, res1, c1, n1);
            c0 = c2;
            n0 = n2;
        }
    }
    if (EPI == EPI_LOGITS) {
        /* first index wins ties: rows are visited in increasing order per
         * wave, waves and WGs own increasing row ranges */
        if (lane == 0) { s_red[wave] = best; s_int[wave] = besti; }
        bar();
        if (threadIdx.x == 0) {
            float bv = s_red[0];
            int bi = s_int[0];
            for (int w = 1; w < PK_WAVES; w++)
                if (s_red[w] > bv || (s_red[w] == bv && s_int[w] < bi)) { bv = s_red[w]; bi = s_int[w]; }
            cst(&P.amax_v[blockIdx.x], bv);
            cst(&P.amax_i[blockIdx.x], bi);
        }
    }
    if (sig) pk_signal(P, sig);
    else if (EPI == EPI_LOGITS) {
        wait_stores();
        bar();
    }
    stamp(tr, 3);
    if (EPI == EPI_LOGITS) {
        if (threadIdx.x == 0) {
            const uint32_t old = __hip_atomic_fetch_add(P.amax_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_int[0] = old == gridDim.x - 1;
        }
        bar();
        if (s_int[0] && threadIdx.x == 0) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int w = 0; w < (int)gridDim.x; w++) {
                const float v = cld(&P.amax_v[w]);
                const int i = cld(&P.amax_i[w]);
                if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
            }
            cst(P.tok_out, bi == 0x7fffffff ? 0 : bi);
            cst(P.amax_cnt, 0u);
        }
    }
}

/* ------------------------------------------------------------------ */
/* attention phase                                                      */
/* ------------------------------------------------------------------ */
/* One head of HD values held 4 per lane (lanes 4l < HD): Qwen3 QK RMSNorm
 * (when nw) and adjacent-pair RoPE, exactly as k_qk_norm_rope_kv. */
template <int HD>
__device__ __forceinline__ void norm_rope_head(float e[4], const float* __restrict__ nw, float eps, int rope_dim,
                                               int pos, const float* __restrict__ freq)
{
    const int lane = threadIdx.x & 63;
    const bool act = 4 * lane < HD;
    if (nw) {
        float ss = e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
        ss = lg_group_sum<64>(ss);
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
        if (act) {
            const float4 g = *(const float4*)(nw + 4 * lane);
            e[0] = e[0] * sc * g.x; e[1] = e[1] * sc * g.y; e[2] = e[2] * sc * g.z; e[3] = e[3] * sc * g.w;
        }
    }
    int rd = rope_dim < HD ? rope_dim : HD;
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
    }
}

/* 8 fp16 values of a cache row (one 16-byte load) as fp32 */
__device__ __forceinline__ void h8(const uint4& v, float f[8])
{
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = lg_h2f((uint16_t)(u[i] & 0xffffu));
        f[2 * i + 1] = lg_h2f((uint16_t)(u[i] >> 16));
    }
}

/* combine two online-softmax states (running max m, sum l, weighted o) */
__device__ __forceinline__ void osm_merge(float& m, float& l, float* o, float m2, float l2, const float* o2, int n)
{
    const float mn = fmaxf(m, m2);
    const float a = m == -INFINITY ? 0.0f : expf(m - mn);
    const float b = m2 == -INFINITY ? 0.0f : expf(m2 - mn);
    l = l * a + l2 * b;
    for (int i = 0; i < n; i++) o[i] = o[i] * a + o2[i] * b;
    m = mn;
}

/* Attention units (kv head g, chunk c of positions [c*chunk, ...) <= pos):
 * one pass over K and V with an online softmax per lane group; LPP lanes
 * hold one position (8 dims each), the step of a workgroup covers
 * PK_WAVES * 64/LPP positions, and the K/V loads of step s+1 are in flight
 * while step s computes (the first step's before the dependency wait: the
 * cache rows < pos do not depend on this token).  With one chunk per head
 * the unit writes att directly; otherwise it writes its (m, l, o) partial
 * and the last unit of the head (atomic counter) merges the partials. */
template <int HD, int NREP>
__device__ __forceinline__ void phase_attn(const PkParams& P, int layer, int pos, int chunk, int nch,
                                           const float* __restrict__ qkv, float* __restrict__ att,
                                           uint64_t wait_target, uint64_t sig, uint64_t* tr)
{
    constexpr int LPP = HD / 8;            /* lanes per position */
    constexpr int PPW = 64 / LPP;          /* positions per wave step */
    constexpr int PPB = PK_WAVES * PPW;    /* positions per WG step */
    const PkLayer& L = P.layers[layer];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane & (LPP - 1), grp = lane / LPP;
    const int kvd = P.kv_dim;
    const int nunits = P.n_kv * nch;
    const size_t loff = (size_t)layer * P.n_ctx * kvd;
    const float scale = 1.0f / sqrtf((float)HD);

    stamp(tr, 0);
    uint4 kb0, vb0, kb1, vb1;   /* K/V of two steps: static names, no indexed registers */
    auto load_step = [&](int u, int st, uint4& kb, uint4& vb) {
        const int g = u / nch, c = u % nch;
        const int t = c * chunk + st * PPB + wave * PPW + grp;
        const int t1 = min(c * chunk + chunk, pos + 1);
        if (t < t1 && t != pos) {
            const size_t o = loff + (size_t)t * kvd + (size_t)g * HD + gl * 8;
            kb = *(const uint4*)(P.kc + o);
            vb = *(const uint4*)(P.vc + o);
        }
    };
    const bool has = (int)blockIdx.x < nunits;
    if (has && (wave != 0 || !wait_target)) load_step(blockIdx.x, 0, kb0, vb0);
    if (wait_target) {
        pk_wait(P, wait_target);
        if (has && wave == 0) load_step(blockIdx.x, 0, kb0, vb0);
    }
    stamp(tr, 1);

    for (int u = blockIdx.x; u < nunits; u += gridDim.x) {
        const int g = u / nch, c = u % nch;
        const int t0 = c * chunk;
        const int t1 = min(t0 + chunk, pos + 1);
        const int nsteps = (t1 - t0 + PPB - 1) / PPB;
        if (u != (int)blockIdx.x) load_step(u, 0, kb0, vb0);
        /* q heads g*NREP.., then k and v of g: normed/roped into LDS */
        for (int h = wave; h <= NREP; h += PK_WAVES) {
            const bool is_q = h < NREP;
            const float* srcp = is_q ? qkv + (size_t)(g * NREP + h) * HD : qkv + P.n_embed + (size_t)g * HD;
            float e[4] = {0.f, 0.f, 0.f, 0.f};
            if (4 * lane < HD) {
                const float4 t = *(const float4*)(srcp + 4 * lane);
                e[0] = t.x; e[1] = t.y; e[2] = t.z; e[3] = t.w;
            }
            norm_rope_head<HD>(e, is_q ? L.q_norm : L.k_norm, P.eps, P.rope_dim, pos, P.rope_freq);
            if (4 * lane < HD) {
                float* dst = is_q ? s_q + h * HD : s_kv;
                *(float4*)(dst + 4 * lane) = make_float4(e[0], e[1], e[2], e[3]);
                if (!is_q) {
                    const float4 vv = *(const float4*)(qkv + P.n_embed + kvd + (size_t)g * HD + 4 * lane);
                    *(float4*)(s_kv + HD + 4 * lane) = vv;
                    if (c == nch - 1) {
                        /* fp16 KV row pos (fast/ligguf_fast_qk.cpp:57-62), read from the next token on */
                        const size_t o = loff + (size_t)pos * kvd + (size_t)g * HD + 4 * lane;
                        const uint32_t klo = (uint32_t)lg_f2h(e[0]) | ((uint32_t)lg_f2h(e[1]) << 16);
                        const uint32_t khi = (uint32_t)lg_f2h(e[2]) | ((uint32_t)lg_f2h(e[3]) << 16);
                        const uint32_t vlo = (uint32_t)lg_f2h(vv.x) | ((uint32_t)lg_f2h(vv.y) << 16);
                        const uint32_t vhi = (uint32_t)lg_f2h(vv.z) | ((uint32_t)lg_f2h(vv.w) << 16);
                        *(uint2*)(P.kc + o) = make_uint2(klo, khi);
                        *(uint2*)(P.vc + o) = make_uint2(vlo, vhi);
                    }
                }
            }
        }
        bar();
        float qr[NREP][8];
#pragma unroll
        for (int r = 0; r < NREP; r++)
#pragma unroll
            for (int i = 0; i < 8; i++) qr[r][i] = s_q[r * HD + gl * 8 + i];

        /* one pass: scores, online softmax, p.V (t == pos uses the fp32 k/v
         * of this step, fast/ligguf_fast_qk.cpp:77-79,98-99) */
        float m[NREP], l[NREP], o[NREP][8];
#pragma unroll
        for (int r = 0; r < NREP; r++) {
            m[r] = -INFINITY;
            l[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) o[r][i] = 0.0f;
        }
        auto step = [&](int st, const uint4& kb, const uint4& vb) {
            const int t = t0 + st * PPB + wave * PPW + grp;
            if (t < t1) {
                float kf[8], vf[8];
                if (t != pos) {
                    h8(kb, kf);
                    h8(vb, vf);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) { kf[i] = s_kv[gl * 8 + i]; vf[i] = s_kv[HD + gl * 8 + i]; }
                }
#pragma unroll
                for (int r = 0; r < NREP; r++) {
                    float sc = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; i++) sc += qr[r][i] * kf[i];
                    sc = lg_group_sum<LPP>(sc) * scale;
                    const float mn = fmaxf(m[r], sc);
                    const float a = expf(m[r] - mn);     /* 0 while m = -inf */
                    const float pw = expf(sc - mn);
                    l[r] = l[r] * a + pw;
#pragma unroll
                    for (int i = 0; i < 8; i++) o[r][i] = o[r][i] * a + pw * vf[i];
                    m[r] = mn;
                }
            }
        };
        /* two steps per iteration, the loads of the next step in flight */
        for (int st = 0; st < nsteps; st += 2) {
            if (st + 1 < nsteps) load_step(u, st + 1, kb1, vb1);
            step(st, kb0, vb0);
            if (st + 2 < nsteps) load_step(u, st + 2, kb0, vb0);
            if (st + 1 < nsteps) step(st + 1, kb1, vb1);
        }
        /* combine the position groups of the wave, then the waves (LDS) */
#pragma unroll
        for (int off = LPP; off < 64; off <<= 1) {
#pragma unroll
            for (int r = 0; r < NREP; r++) {
                float o2[8];
#pragma unroll
                for (int i = 0; i < 8; i++) o2[i] = __shfl_xor(o[r][i], off, 64);
                const float m2 = __shfl_xor(m[r], off, 64), l2 = __shfl_xor(l[r], off, 64);
                osm_merge(m[r], l[r], o[r], m2, l2, o2, 8);
            }
        }
        if (grp == 0) {
#pragma unroll
            for (int r = 0; r < NREP; r++) {
#pragma unroll
                for (int i = 0; i < 8; i++) s_o[(wave * NREP + r) * HD + gl * 8 + i] = o[r][i];
                if (gl == 0) { s_m[wave * NREP + r] = m[r]; s_sc[wave * NREP + r] = l[r]; }
            }
        }
        bar();
        const bool direct = nch == 1;
        float* part = P.attn_ws + (size_t)u * NREP * (HD + 2);
        for (int i = threadIdx.x; i < NREP * HD; i += PK_THREADS) {
            const int r = i / HD;
            float M = s_m[r], Ls = s_sc[r], O = s_o[r * HD + i % HD];
            for (int w = 1; w < PK_WAVES; w++) {
                const float o2 = s_o[(w * NREP + r) * HD + i % HD];
                osm_merge(M, Ls, &O, s_m[w * NREP + r], s_sc[w * NREP + r], &o2, 1);
            }
            if (direct) cst(&att[(size_t)g * NREP * HD + i], O / Ls);
            else {
                cst(&part[2 * NREP + i], O);
                if (i % HD == 0) { cst(&part[r], M); cst(&part[NREP + r], Ls); }
            }
        }
        if (!direct) {
            wait_stores();
            bar();
            if (threadIdx.x == 0) {
                const uint32_t old = __hip_atomic_fetch_add(&P.attn_cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_int[0] = old == (uint32_t)(nch - 1);
            }
            bar();
            if (s_int[0]) {
                /* last unit of head group g: merge its nch partials.  (m, l)
                 * of all chunks go through LDS; each thread then sums one
                 * output value over the chunks with 8 loads in flight. */
                constexpr int ST = NREP * (HD + 2);
                const float* base = P.attn_ws + (size_t)g * nch * ST;
                float* s_ml = s_sc;                                   /* [nch][2*NREP]: m then l */
                float* s_w = s_sc + PK_MAX_UNITS_PER_HEAD * 2 * NREP; /* [nch][NREP] weights */
                for (int i = threadIdx.x; i < nch * 2 * NREP; i += PK_THREADS)
                    s_ml[i] = cld(&base[(size_t)(i / (2 * NREP)) * ST + i % (2 * NREP)]);
                bar();
                if (threadIdx.x < NREP) {
                    const int r = threadIdx.x;
                    float M = -INFINITY;
                    for (int cc = 0; cc < nch; cc++) M = fmaxf(M, s_ml[cc * 2 * NREP + r]);
                    float Ls = 0.0f;
                    for (int cc = 0; cc < nch; cc++) {
                        const float wgt = expf(s_ml[cc * 2 * NREP + r] - M);
                        s_w[cc * NREP + r] = wgt;
                        Ls += s_ml[cc * 2 * NREP + NREP + r] * wgt;
                    }
                    s_red[r] = Ls;
                }
                bar();
                for (int i = threadIdx.x; i < NREP * HD; i += PK_THREADS) {
                    const int r = i / HD;
                    float acc = 0.0f;
                    for (int c0 = 0; c0 < nch; c0 += 8) {
                        float v[8];
#pragma unroll
                        for (int k = 0; k < 8; k++)
                            v[k] = c0 + k < nch ? cld(&base[(size_t)(c0 + k) * ST + 2 * NREP + i]) : 0.0f;
#pragma unroll
                        for (int k = 0; k < 8; k++)
                            if (c0 + k < nch) acc += v[k] * s_w[(c0 + k) * NREP + r];
                    }
                    cst(&att[(size_t)g * NREP * HD + i], acc / s_red[r]);
                }
                if (threadIdx.x == 0) cst(&P.attn_cnt[g], 0u);
            }
        }
        bar();
    }
    stamp(tr, 2);
    if (sig) pk_signal(P, sig);
    stamp(tr, 3);
}


/* ------------------------------------------------------------------ */
/* work sizes                                                           */
/* ------------------------------------------------------------------ */
/* rows of one item held per lane: enough items in flight to cover the wait,
 * within a register budget of ~144 VGPRs for the weights */
template <int FMT, int NS, int K, int CAP, int BUDGET = 576>
struct Batch {
    static constexpr int bytes = (int)sizeof(typename Fmt<FMT>::W) * NS * K;
    static constexpr int v = BUDGET / bytes;
    static constexpr int value = v < 1 ? 1 : (v > CAP ? CAP : v);
};

/* slots per lane at width n_embed = 4096: one 64-value slot, two Q8_0 slots */
template <int T>
struct NsE {
    static constexpr int value = T == LG_Q8_0 ? 2 : 1;
};

