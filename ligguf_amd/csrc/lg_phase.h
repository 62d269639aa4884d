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

/* thread index in the workgroup as the phases read it.  A kernel that walks
 * all layers with every phase inlined defines LG_TID before including this
 * header as an index the compiler cannot see through: otherwise it hoists the
 * per-lane address arithmetic of every phase out of the layer loop and keeps
 * it live (spilled) across the whole loop. */
#ifndef LG_TID
#define LG_TID ((int)threadIdx.x)
#endif

/* matvec phases: wave w of the grid takes items w, w + waves, w + 2 waves, ...
 * so that all waves sweep each window of consecutive rows together (DRAM
 * pages and channels see one moving window); 0 = a contiguous range per wave */
#ifndef LG_MV_SPREAD
#define LG_MV_SPREAD 1
#endif

/* ------------------------------------------------------------------ */
/* LDS                                                                  */
/* ------------------------------------------------------------------ */
/* activation build area: fp32 staging of x (rmsnorm) + quantized blocks */
__shared__ __attribute__((aligned(16))) float s_x[PK_MAX_EMBED];
__shared__ __attribute__((aligned(16))) uint8_t s_act[(PK_MAX_FF / 256) * LG_BS_Q8_K + 64];
/* the fp32 activation of F16 / F32 rows, each 32-value slot followed by 4 unused
 * floats: lanes read consecutive slots, and a 144-byte slot stride puts
 * their 16-byte reads on distinct banks (a 128-byte stride would put every
 * lane on the same ones).  Kernels of other formats do not reference it, so
 * it takes LDS in F16 kernels only. */
#define PK_ACTF_SLOT 36
__shared__ __attribute__((aligned(16))) float s_actf[PK_MAX_FF_F / 32 * PK_ACTF_SLOT];
__shared__ float s_red[64];
__shared__ int s_int[8];
/* attention */
__shared__ __attribute__((aligned(16))) float s_q[PK_MAX_NREP * 128];
__shared__ __attribute__((aligned(16))) float s_kv[2 * 128];
__shared__ __attribute__((aligned(16))) float s_sc[3 * PK_ATT_MAX_NCH * PK_MAX_NREP];
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

/* keeps the loads before it ahead of the loads after it in issue order (a
 * wave's loads return in issue order, so what is needed first is issued
 * first); no wait is implied */
__device__ __forceinline__ void lg_issue_order()
{
    asm volatile("" ::: "memory");
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
    if (LG_TID == 0) cst(&P.progress[blockIdx.x], val);
}

/* wait until every WG's progress word reaches `target` (wave 0 polls) */
__device__ __forceinline__ void pk_wait(const PkParams& P, uint64_t target)
{
    if (LG_TID < 64) {
        if (!cld(P.err)) {
            const int nwg = gridDim.x;
            bool ok = false;
            int it = 0;
            do {
                uint64_t mn = ~0ull;
                for (int i = LG_TID; i < nwg; i += 64) {
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
            if (!ok && LG_TID == 0) cst(P.err, 1u);
        }
    }
    bar();
}

/* KV-group barrier of the fused QKV + attention kernel.  Each workgroup of
 * a group owns one word of the group's gsz consecutive words and counts its
 * launches in it: it reads its word at kernel start (group_round), stores
 * the incremented value once its rows are stored (group_arrive: stores
 * acknowledged first, as pk_signal), and waits until every word of the
 * group holds at least that value (group_wait: one load per lane, wave 0;
 * bounded by spin_cap, past which P.err is set, as pk_wait).  Every
 * workgroup arrives once per launch, so the words advance in step. */
__device__ __forceinline__ uint64_t group_round(const uint64_t* mine)
{
    return cld(mine) + 1;
}

__device__ __forceinline__ void group_arrive(uint64_t* mine, uint64_t round)
{
    wait_stores();
    bar();
    if (LG_TID == 0) cst(mine, round);
}

__device__ __forceinline__ void group_wait(const PkParams& P, const uint64_t* words, int gsz, uint64_t round)
{
    if (LG_TID < 64) {
        bool ok = false;
        int it = 0;
        do {
            uint64_t mn = ~0ull;
            for (int i = LG_TID; i < gsz; i += 64) {
                const uint64_t v = cld(&words[i]);
                mn = v < mn ? v : mn;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const uint64_t t = __shfl_xor(mn, o, 64);
                mn = t < mn ? t : mn;
            }
            ok = mn >= round;
        } while (!ok && ++it < P.spin_cap);
        if (!ok && LG_TID == 0) cst(P.err, 1u);
    }
    bar();
}

/* the online softmax moves its reference max only past this margin (log2
 * units): the running sums are rescaled then, not at every new maximum */
#define PK_ATT_LAZY 8.0f

/* lg_group_sum of N values, each butterfly step over all of them in turn */
template <int G, int N>
__device__ __forceinline__ void lg_group_sum_n(float* v)
{
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 2) v[r] += lg_partner<0>(v[r]);
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 4) v[r] += lg_partner<1>(v[r]);
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 8) v[r] += lg_partner<2>(v[r]);
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 16) v[r] += lg_partner<3>(v[r]);
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 32) v[r] += lg_partner<4>(v[r]);
#pragma unroll
    for (int r = 0; r < N; r++) if constexpr (G >= 64) v[r] += lg_partner<5>(v[r]);
}

/* 2^x (v_exp_f32): attention scores are kept in log2 units */
__device__ __forceinline__ float lg_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

/* phase timestamps (lane 0 of wave 0 of every WG; nothing when tr is NULL).
 * The store goes through the global address space: a flat store would also
 * count against lgkmcnt and make the next LDS wait wait for it. */
__device__ __forceinline__ void stamp(uint64_t* tr, int k)
{
    if (tr && LG_TID == 0) *(__attribute__((address_space(1))) uint64_t*)(tr + k) = wall_clock64();
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
/* BLD_RMS: rmsnorm of the source vector; BLD_EMB: rmsnorm of the embedding
 * row; BLD_PLAIN: the source vector as it is; BLD_MERGE: the attention
 * partials merged (MergeSrc); BLD_KEEP: the activation the previous sweep of
 * the same kernel left in LDS (a second matrix on the same input) */
/* BLD_RSUM: rmsnorm of x + the att_out group partials (PartSum), that sum
 * stored by workgroup 0 as the residual stream xm */
enum { BLD_RMS = 0, BLD_PLAIN = 1, BLD_MERGE = 2, BLD_EMB = 3, BLD_KEEP = 4, BLD_RSUM = 5 };

/* the activation format a weight format's dot reads: Q8_0 blocks for
 * Q8_0/Q1_0/Q1_G rows, Q8_K blocks for the K-quants, fp32 for F16 / F32 rows
 * (the reference's matmul passes the float vector to dot_f16_f32 / dot_f32,
 * fast/lil_math.cpp:397-409) */
__host__ __device__ constexpr int lg_act_qt(int fmt)
{
    return (fmt == LG_F16_L || fmt == LG_F32_L) ? LG_F32
         : (fmt == LG_Q8_0 || fmt == LG_Q8_0_R || fmt == LG_Q1_0 || fmt == LG_Q1_0_R || fmt == LG_Q1_G ||
            fmt == LG_Q1_G_R) ? LG_Q8_0 : LG_Q8_K;
}

/* the wave's 256 values of chunk ch as an activation of format QT: fp32
 * into s_actf (slot-padded), quantized blocks into s_act */
template <int QT>
__device__ __forceinline__ void act_emit(const float v[4], int ch, int nvalid)
{
    if constexpr (QT == LG_F32) {
        const int lane = LG_TID & 63;
        if (4 * lane < nvalid)
            *(float4*)(s_actf + ch * (8 * PK_ACTF_SLOT) + (lane >> 3) * PK_ACTF_SLOT + 4 * (lane & 7)) =
                make_float4(v[0], v[1], v[2], v[3]);
    } else {
        lg_emit(v, QT, s_act, ch, nvalid);
    }
}

/* F16 rows against the fp32 activation in s_actf: the slot's 32 floats are
 * read from LDS at each dot (held in registers they would take 32 VGPRs a
 * slot, 192 for a 12288-value down row), the same products and order as
 * Fmt<LG_F16> (dot_f16_f32, fast/arch_avx2.h:83-109) */
template <>
struct Fmt<LG_F16_L> {
    static constexpr int VALS = 32;
    struct Act {
        int s;
    };
    using W = Fmt<LG_F16>::W;
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t*, int s) { A.s = s; }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s) { Fmt<LG_F16>::load_w(w, row, s); }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        const float4* a = (const float4*)(s_actf + A.s * PK_ACTF_SLOT);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 p = a[2 * i], q = a[2 * i + 1];
            const float f[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
            const uint32_t u[4] = {w.v[i].x, w.v[i].y, w.v[i].z, w.v[i].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc += lg_h2f((uint16_t)(u[k] & 0xffffu)) * f[2 * k];
                acc += lg_h2f((uint16_t)(u[k] >> 16)) * f[2 * k + 1];
            }
        }
        return acc;
    }
};

/* F32 rows against the same fp32 activation: the products and order of
 * Fmt<LG_F32> (dot_f32, fast/arch_avx2.h:83-109) */
template <>
struct Fmt<LG_F32_L> {
    static constexpr int VALS = 32;
    using Act = Fmt<LG_F16_L>::Act;
    using W = Fmt<LG_F32>::W;
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t*, int s) { A.s = s; }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s) { Fmt<LG_F32>::load_w(w, row, s); }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        const float4* a = (const float4*)(s_actf + A.s * PK_ACTF_SLOT);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = a[i];
            acc += __builtin_fmaf(w.v[i].w, f.w, __builtin_fmaf(w.v[i].z, f.z, lg_fma2(w.v[i].x, f.x, w.v[i].y, f.y)));
        }
        return acc;
    }
};

__device__ __forceinline__ int chunk_base(int c)
{
    return ((LG_TID >> 6) + PK_WAVES * c) * 256 + 4 * (LG_TID & 63);
}

/* an activation of width n below the CPW * 256 * PK_WAVES a build covers:
 * loads past n read its last four values (unconditional loads), and those
 * values count as zero */
__device__ __forceinline__ int chunk_ld(int c, int n)
{
    const int b = chunk_base(c);
    return b < n ? b : n - 4;
}

/* rmsnorm weights of this wave's chunks: constants, loaded before the wait */
template <int CPW>
struct NormW {
    float4 g[CPW];
    __device__ __forceinline__ void load(const float* __restrict__ w, int n)
    {
#pragma unroll
        for (int c = 0; c < CPW; c++) g[c] = *(const float4*)(w + chunk_ld(c, n));
    }
};

/* this wave's chunks of an activation source vector, loaded on their own
 * so that they can be issued ahead of the weight loads (a wave's loads
 * return in issue order) */
template <int CPW>
struct ActSrc {
    float4 v[CPW];
    __device__ __forceinline__ void load(const float* __restrict__ src, int n)
    {
#pragma unroll
        for (int c = 0; c < CPW; c++) v[c] = *(const float4*)(src + chunk_ld(c, n));
    }
};

/* The att_out rows split by KV group (the fused QKV + attention + att_out
 * kernel): group g's partial of row i is the sum of the row's slots 8g ..
 * 8g+7 -- lanes 8g .. 8g+7 of a whole-row dot, whose lg_wave_sum adds the
 * aligned 8-lane groups g0..g7 as ((g6+g7)+(g4+g5)) + ((g2+g3)+(g0+g1)).
 * The sum below adds the 8 partials of each value in that order and then
 * the residual, as EPI_RESID adds res + the wave sum, so xm comes out bit
 * for bit as the att_out phase computes it.  part: [8][n] */
template <int CPW>
struct PartSum {
    float4 p[8][CPW];
    __device__ __forceinline__ void load(const float* __restrict__ part, int n)
    {
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int c = 0; c < CPW; c++) p[k][c] = *(const float4*)(part + (size_t)k * n + chunk_ld(c, n));
    }
    __device__ __forceinline__ static float tree(float a0, float a1, float a2, float a3, float a4, float a5, float a6,
                                                 float a7)
    {
        return ((a6 + a7) + (a4 + a5)) + ((a2 + a3) + (a0 + a1));
    }
    /* x + the partials, in place */
    __device__ __forceinline__ void add_to(ActSrc<CPW>& x) const
    {
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            float4& v = x.v[c];
            v.x = v.x + tree(p[0][c].x, p[1][c].x, p[2][c].x, p[3][c].x, p[4][c].x, p[5][c].x, p[6][c].x, p[7][c].x);
            v.y = v.y + tree(p[0][c].y, p[1][c].y, p[2][c].y, p[3][c].y, p[4][c].y, p[5][c].y, p[6][c].y, p[7][c].y);
            v.z = v.z + tree(p[0][c].z, p[1][c].z, p[2][c].z, p[3][c].z, p[4][c].z, p[5][c].z, p[6][c].z, p[7][c].z);
            v.w = v.w + tree(p[0][c].w, p[1][c].w, p[2][c].w, p[3][c].w, p[4][c].w, p[5][c].w, p[6][c].w, p[7][c].w);
        }
    }
};

/* attention partials of one layer, merged by the att_out build (BLD_MERGE):
 * the source vector is sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c,
 * M = max_c m_c, over the nch chunks in ascending order */
struct MergeSrc {
    const float* po;     /* [nch][n_embed] */
    const float* pml;    /* [nch][n_heads][2] */
    int nch;             /* 1..PK_ATT_MERGE */
    int head_dim;
};

template <int CPW>
struct MergeAct {
    float4 o[PK_ATT_MERGE][CPW];
    float2 ml[PK_ATT_MERGE][CPW];

    __device__ __forceinline__ void load(const MergeSrc& ms, int ne, int nh)
    {
#pragma unroll
        for (int c = 0; c < PK_ATT_MERGE; c++) {
            const int cc = min(c, ms.nch - 1);   /* unconditional loads (see Rows) */
#pragma unroll
            for (int k = 0; k < CPW; k++) {
                const int b = chunk_ld(k, ne);
                o[c][k] = *(const float4*)(ms.po + (size_t)cc * ne + b);
                ml[c][k] = *(const float2*)(ms.pml + ((size_t)cc * nh + b / ms.head_dim) * 2);
            }
        }
    }

    /* CPW = 1: the four values at b (b = chunk * 256 + 4 * lane) of an
     * explicitly named chunk, loaded as load() loads the wave's own */
    __device__ __forceinline__ void load_at(const MergeSrc& ms, int nh, int ne, int b)
    {
        static_assert(CPW == 1, "one chunk");
#pragma unroll
        for (int c = 0; c < PK_ATT_MERGE; c++) {
            const int cc = min(c, ms.nch - 1);
            o[c][0] = *(const float4*)(ms.po + (size_t)cc * ne + b);
            ml[c][0] = *(const float2*)(ms.pml + ((size_t)cc * nh + b / ms.head_dim) * 2);
        }
    }

    __device__ __forceinline__ void merge(int nch, ActSrc<CPW>& a) const
    {
#pragma unroll
        for (int k = 0; k < CPW; k++) {
            float M = ml[0][k].x;
#pragma unroll
            for (int c = 1; c < PK_ATT_MERGE; c++)
                if (c < nch) M = fmaxf(M, ml[c][k].x);
            float Ls = 0.0f;
            float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int c = 0; c < PK_ATT_MERGE; c++) {
                if (c < nch) {
                    const float w = lg_exp2(ml[c][k].x - M);
                    Ls += ml[c][k].y * w;
                    O.x += o[c][k].x * w; O.y += o[c][k].y * w; O.z += o[c][k].z * w; O.w += o[c][k].w * w;
                }
            }
            const float inv = 1.0f / Ls;
            a.v[k] = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
        }
    }
};

#ifndef LG_ATT_H2
#define LG_ATT_H2 2
#endif

/* long-context chunks per head: the attention grid's workgroups per head
 * group (the same for the fused and the persistent step) */
__device__ __forceinline__ int pk_att_max_nch(const PkParams& P)
{
    return P.att_grid / P.n_kv;
}

/* the attention partials of layer l at position pos as the att_out build
 * reads them: the fixed chunks (short contexts), the chunks of
 * pk_attn_split, or past PK_ATT_MERGE of those their group slots */
template <int HD, int NREP>
__device__ __forceinline__ MergeSrc att_partials(const PkParams& P, int l, int pos)
{
    int chunk, nch;
    if (!pk_att_long(pos, HD, NREP, P.n_kv, gridDim.x)) {
        chunk = pk_att_fch(HD, NREP);
        nch = (pos + chunk) / chunk;
    } else {
        pk_attn_split(pos + 1, HD, NREP, pk_att_max_nch(P), &chunk, &nch);
    }
    const bool grp = nch > PK_ATT_MERGE;
    const size_t slot = (size_t)l * P.att_slots + (grp ? P.att_slots - PK_ATT_MERGE : 0);
    return MergeSrc{P.att_po + slot * P.n_embed, P.att_pml + slot * P.n_heads * 2,
                    grp ? pk_att_ngroups(nch) : nch, HD};
}

/* rmsnorm(x) * w quantized into s_act (fast/lil_math.cpp:922-929 and
 * quantize_q8_K / quantize_q8_0, :329-394).  The sum of squares is taken in
 * the order of k_rmsnorm_quant: per wave over its chunks (lane partials in
 * chunk order, then lg_wave_sum), the wave sums added in wave order -- so
 * both paths agree bit for bit.  x is the source vector (BLD_RMS) or, for
 * layer 0 (BLD_EMB), the embedding row of tok, dequantized here; WG 0 also
 * stores that row as the residual stream `emb_out`. */
template <int QT, int CPW>
__device__ __forceinline__ void build_rms(const PkParams& P, int tok, const NormW<CPW>& nw, const ActSrc<CPW>& xsrc,
                                          bool from_embed, float* __restrict__ emb_out, int n)
{
    const int lane = LG_TID & 63, wave = LG_TID >> 6;
    float4 xv[CPW];
    if (from_embed) {
        /* one dequantization loop (the switch over types stays out of the
         * unrolled chunk code), staged through s_x */
        const uint8_t* row = P.embd + (size_t)tok * P.embd_rsz;
        for (int i = LG_TID; i < n; i += PK_THREADS) s_x[i] = lg_dq_value(P.embd_t, row, i);
        bar();
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            const int b = chunk_base(c);
            xv[c] = *(const float4*)(s_x + chunk_ld(c, n));
            if (blockIdx.x == 0 && b < n) {
                cst(&emb_out[b], xv[c].x); cst(&emb_out[b + 1], xv[c].y);
                cst(&emb_out[b + 2], xv[c].z); cst(&emb_out[b + 3], xv[c].w);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPW; c++) xv[c] = xsrc.v[c];
    }
#pragma unroll
    for (int c = 0; c < CPW; c++)
        if (chunk_base(c) >= n) xv[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    float p = 0.0f;
#pragma unroll
    for (int c = 0; c < CPW; c++) p += lg_sq4(xv[c]);
    p = lg_wave_sum(p);
    if (lane == 0) s_red[wave] = p;
    bar();
    float ss = 0.0f;
#pragma unroll
    for (int w = 0; w < PK_WAVES; w++) ss += s_red[w];
    const float scale = 1.0f / sqrtf(ss / (float)n + P.eps);
#pragma unroll
    for (int c = 0; c < CPW; c++) {
        const int ch = wave + PK_WAVES * c;
        if (256 * ch >= n) break;   /* wave-uniform */
        const float4 t = xv[c], g = nw.g[c];
        const float v[4] = {t.x * scale * g.x, t.y * scale * g.y, t.z * scale * g.z, t.w * scale * g.w};
        act_emit<QT>(v, ch, min(256, n - 256 * ch));
    }
    bar();
}

/* the source chunks quantized into s_act (fp32 into s_actf) */
template <int QT, int CPW>
__device__ __forceinline__ void build_plain(const ActSrc<CPW>& a, int n)
{
    const int wave = LG_TID >> 6;
#pragma unroll
    for (int c = 0; c < CPW; c++) {
        const int ch = wave + PK_WAVES * c;
        if (256 * ch >= n) break;   /* wave-uniform */
        const bool ok = chunk_base(c) < n;
        const float v[4] = {ok ? a.v[c].x : 0.f, ok ? a.v[c].y : 0.f, ok ? a.v[c].z : 0.f, ok ? a.v[c].w : 0.f};
        act_emit<QT>(v, ch, min(256, n - 256 * ch));
    }
    bar();
}

/* ------------------------------------------------------------------ */
/* matvec phases                                                        */
/* ------------------------------------------------------------------ */
/* The grid's greedy row from the per-workgroup partials (P.amax_v/amax_i
 * [0, n)): the largest value, the lowest row among equal ones -- an
 * order-free rule, so the NT threads of the calling workgroup reduce the
 * partials in parallel (strided loads, then lanes, then waves).  Every
 * thread calls it; thread 0 gets the row (0x7fffffff when no value is a
 * number). */
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i)
{
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

template <int NT>
__device__ __forceinline__ int argmax_partials(const PkParams& P, int n)
{
    __shared__ float s_av[NT / 64];
    __shared__ int s_ai[NT / 64];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int w = (int)threadIdx.x; w < n; w += NT) argmax_take(bv, bi, cld(&P.amax_v[w]), cld(&P.amax_i[w]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_take(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    if ((threadIdx.x & 63) == 0) { s_av[threadIdx.x >> 6] = bv; s_ai[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < NT / 64; w++) argmax_take(bv, bi, s_av[w], s_ai[w]);
    return bi;
}

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

/* Items of one phase are split evenly over all waves of the grid in
 * contiguous runs; an item is K rows (K = 2 for up|gate: rows i and i+kstride)
 * each dotted by the whole wave (lane j owns slots j, j+64, ...).
 *
 * Every load of the hot path is unconditional (indices clamped to a valid
 * item instead of a branch around the load): the compiler counts the loads
 * still in flight with vmcnt, and where a load sits under a branch it must
 * assume the shorter path and wait for every later load as well -- the
 * activation build would then wait for all the wave's weights. */
/* The items of a matvec phase as matrix rows (and output indices): the
 * identity, or (a phase restricted to one KV group's rows) up to three row
 * ranges back to back -- n0 rows from b0, n1 from b1, the rest from b2. */
struct RowMap {
    int n0, b0, n1, b1, b2;   /* n0 < 0: the identity */
    __device__ __forceinline__ int row(int i) const
    {
        if (n0 < 0) return i;
        return i < n0 ? b0 + i : (i < n0 + n1 ? b1 + (i - n0) : b2 + (i - n0 - n1));
    }
};
#define LG_ROWS_ALL (RowMap{-1, 0, 0, 0, 0})

/* The waves that share a phase's items: the whole grid (nwv = 0), or nwv
 * waves of which this workgroup's wave 0 is number gw0 */
struct WaveSet {
    int gw0, nwv;
};
#define LG_WAVES_ALL (WaveSet{0, 0})

template <int FMT, int NS, int MAXB, int K>
struct Rows {
    typename Fmt<FMT>::W w[MAXB][K][NS];

    /* items i0, i0+ist, ... (MAXB of them), those past `wlast` replaced by
     * wlast; slots past the row's nslots read its last slot (not used) */
    __device__ __forceinline__ void load(const uint8_t* __restrict__ W, uint32_t rsz, int i0, int ist, int wlast,
                                         int kstride, int lane, int nslots, const RowMap& rm)
    {
#pragma unroll
        for (int b = 0; b < MAXB; b++) {
            const int i = rm.row(min(i0 + b * ist, wlast));
#pragma unroll
            for (int k = 0; k < K; k++) {
                const uint8_t* row = W + (size_t)(i + k * kstride) * rsz;
#pragma unroll
                for (int s = 0; s < NS; s++) Fmt<FMT>::load_w(w[b][k][s], row, min(lane + 64 * s, nslots - 1));
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
 * store, publish.  CPW = 256-value activation chunks per wave; NR = batches
 * of MAXB items held at once: 1 = load a batch, then compute it; NR >= 2 = a
 * ring in which NR - 1 batches load while one computes (the first NR - 1
 * batches load before the build).  rot shifts the item-to-wave mapping by
 * that many waves (a second sweep starts on the waves the first left with
 * fewer items). */
template <int FMT, int NS, int MAXB, int K, int EPI, int BLD, int CPW, int NR>
__device__ __forceinline__ void phase_mv(const PkParams& P, int tok, const uint8_t* __restrict__ W, uint32_t rsz,
                                         int items, int kstride, const float* __restrict__ normw,
                                         const float* __restrict__ src, const float* __restrict__ res_src,
                                         float* __restrict__ out, float* __restrict__ emb_out,
                                         uint64_t wait_target, uint64_t sig, uint64_t* tr, uint8_t* atr, int n_act,
                                         const MergeSrc& ms = MergeSrc{nullptr, nullptr, 0, 0}, int rot = 0,
                                         const RowMap& rm = LG_ROWS_ALL, const WaveSet& wset = LG_WAVES_ALL)
{
    using F = Fmt<FMT>;
    constexpr int QT = lg_act_qt(FMT);
    /* a row of n_act values is nslots slots; lane j takes slots j, j+64, ..
     * (NS of them, those past nslots unused) */
    const int nslots = n_act / F::VALS;
    /* the wave index as a wave-uniform value: item indices and row addresses
     * are then scalar (a row base in SGPRs, the lane's slot offset in a VGPR) */
    const int lane = LG_TID & 63, wave = __builtin_amdgcn_readfirstlane(LG_TID >> 6);
    const int nwv = wset.nwv ? wset.nwv : gridDim.x * PK_WAVES;
    int gw = (wset.nwv ? wset.gw0 : blockIdx.x * PK_WAVES) + wave + rot;   /* 0 <= rot < nwv */
    gw -= gw >= nwv ? nwv : 0;
#if LG_MV_SPREAD
    const int ist = nwv, i0 = gw;
    const int my = gw < items ? (items - gw + nwv - 1) / nwv : 0;
#else
    const int ipw = (items + nwv - 1) / nwv;
    const int ist = 1, i0 = gw * ipw;
    const int my = max(0, min(items, i0 + ipw) - i0);
#endif
    const int wlast = my > 0 ? i0 + (my - 1) * ist : items - 1;   /* clamp for the loads */

    stamp(tr, 0);
    static_assert(NR >= 1 && NR <= 4, "ring depth");
    Rows<FMT, NS, MAXB, K> R[NR];
    /* EPI_RESID: lane j holds the residual of the wave's item j (of the
     * current 64-item chunk; items past the wave's last load its last) */
    float resl = 0.0f;
    NormW<CPW> nw;
    ActSrc<CPW> as;
    MergeAct<CPW> mg;
    constexpr bool from_embed = BLD == BLD_EMB;
    constexpr bool rms = BLD == BLD_RMS || BLD == BLD_EMB || BLD == BLD_RSUM;
    PartSum<BLD == BLD_RSUM ? CPW : 1> ps;
    auto load_src = [&]() {
        if (BLD == BLD_MERGE) mg.load(ms, P.n_embed, P.n_heads);
        else if (!from_embed && BLD != BLD_KEEP) as.load(src, n_act);
        if (BLD == BLD_RSUM) ps.load(P.ao_part, n_act);
    };
    auto load_res = [&](int c0) {
        if (EPI == EPI_RESID) resl = res_src[rm.row(min(i0 + (c0 + lane) * ist, wlast))];
    };
    auto prefetch = [&]() {
#pragma unroll
        for (int k = 0; k < (NR > 1 ? NR - 1 : 1); k++)
            R[k].load(W, rsz, i0 + k * MAXB * ist, ist, wlast, kstride, lane, nslots, rm);
        load_res(0);
    };
    if (!wait_target) {
        /* no dependency wait (fused kernels): the activation and the norm
         * weights go first, the rows after them */
        load_src();
        if (rms) nw.load(normw, n_act);
        lg_issue_order();   /* activation first */
        prefetch();
    } else {
        if (rms) nw.load(normw, n_act);
        if (wave != 0) prefetch();
        pk_wait(P, wait_target);
        load_src();
        if (wave == 0) prefetch();
    }
    stamp(tr, 1);
    if constexpr (BLD == BLD_RSUM) {
        /* xm = x + the att_out group partials; workgroup 0 stores it (the
         * down phase's residual) */
        ps.add_to(as);
        if (blockIdx.x == 0) {
#pragma unroll
            for (int c = 0; c < CPW; c++)
                if (chunk_base(c) < n_act) *(float4*)(emb_out + chunk_base(c)) = as.v[c];
        }
    }
    if (rms) build_rms<QT, CPW>(P, tok, nw, as, from_embed, emb_out, n_act);
    else if (BLD != BLD_KEEP) {
        if (BLD == BLD_MERGE) mg.merge(ms.nch, as);
        build_plain<QT, CPW>(as, n_act);
    }
    stamp(tr, 2);
    if (QT != LG_F32 && atr && blockIdx.x == 0) {
        /* activation trace (tests): the quantized blocks as built (fp32
         * activations are not compared: nothing is quantized there) */
        const int words = ((QT == LG_Q8_K ? n_act / 256 * LG_BS_Q8_K : n_act / 32 * LG_BS_Q8_0) + 3) / 4;
        for (int i = LG_TID; i < words; i += PK_THREADS) ((uint32_t*)atr)[i] = ((const uint32_t*)s_act)[i];
    }

    typename F::Act act[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) F::load_act(act[s], s_act, min(lane + 64 * s, nslots - 1));

    /* Item results gather in lanes -- lane j holds the wave's item c0 + j
     * (ov; og the gate row's for EPI_SWIGLU) -- and every 64 items, and
     * after the last, all lanes finish their items at once: one epilogue and
     * one store instruction per 64 items instead of a lane-0 epilogue per
     * item (the same arithmetic per item). */
    float ov = 0.0f, og = 0.0f;
    float best = -INFINITY;   /* EPI_LOGITS: this lane's best item so far, first index on ties */
    int besti = 0x7fffffff;
    int c0 = 0;
    auto flush = [&](int n) {
        if (lane < n) {
            const int i = rm.row(i0 + (c0 + lane) * ist);
            float v = ov;
            if (EPI == EPI_RESID) v = resl + ov;
            else if (EPI == EPI_SWIGLU) v = (og / (1.0f + expf(-og))) * ov;
            if (EPI == EPI_LOGITS) {
                out[i] = v;
                if (v > best) { best = v; besti = i; }
            } else {
                cst(&out[i], v);
            }
        }
        c0 += 64;
        if (c0 < my) load_res(c0);
    };
    auto process = [&](const Rows<FMT, NS, MAXB, K>& R, int b0, int nb) {
#pragma unroll
        for (int b = 0; b < MAXB; b++) {
            if (b < nb) {
                float acc[K];
#pragma unroll
                for (int k = 0; k < K; k++) {
                    float a = 0.0f;
#pragma unroll
                    for (int s = 0; s < NS; s++)
                        if (64 * (s + 1) <= nslots || lane + 64 * s < nslots) a += F::dot(R.w[b][k][s], act[s], lane + 64 * s);
                    acc[k] = lg_wave_sum(a);
                }
                const int li = b0 + b - c0;   /* wave-uniform */
                ov = lane == li ? acc[0] : ov;
                if (EPI == EPI_SWIGLU) og = lane == li ? acc[1] : og;
                if (li == 63) flush(64);
            }
        }
    };
    if (NR == 1) {
        for (int b0 = 0; b0 < my; b0 += MAXB) {
            if (b0 > 0) R[0].load(W, rsz, i0 + b0 * ist, ist, wlast, kstride, lane, nslots, rm);
            process(R[0], b0, min(MAXB, my - b0));
        }
    } else {
        /* batch j sits in slot j % NR; before computing batch j the wave
         * issues batch j + NR - 1 into the slot batch j - 1 freed (past the
         * end: clamped duplicates of its last row, never used) */
        for (int j0 = 0; j0 * MAXB < my; j0 += NR) {
#pragma unroll
            for (int k = 0; k < NR; k++) {
                const int jn = j0 + k + NR - 1;
                R[(k + NR - 1) % NR].load(W, rsz, i0 + jn * MAXB * ist, ist, wlast, kstride, lane, nslots, rm);
                process(R[k], (j0 + k) * MAXB, min(MAXB, my - (j0 + k) * MAXB));
            }
        }
    }
    if (my > c0) flush(my - c0);
    if (EPI == EPI_LOGITS) {
        /* the wave's best: the largest value, the lowest row index among
         * equal ones (each lane's best is its first among equal values; its
         * rows ascend) */
        float mx = best;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        int mi = best == mx ? besti : 0x7fffffff;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mi = min(mi, __shfl_xor(mi, o, 64));
        best = mx;
        besti = mi;
    }
    if (EPI == EPI_LOGITS) {
        /* first index wins ties: rows are visited in increasing order per
         * wave, waves and WGs own increasing row ranges */
        if (lane == 0) { s_red[wave] = best; s_int[wave] = besti; }
        bar();
        if (LG_TID == 0) {
            float bv = s_red[0];
            int bi = s_int[0];
            for (int w = 1; w < PK_WAVES; w++)
                if (s_red[w] > bv || (s_red[w] == bv && s_int[w] < bi)) { bv = s_red[w]; bi = s_int[w]; }
            cst(&P.amax_v[blockIdx.x], bv);
            cst(&P.amax_i[blockIdx.x], bi);
        }
    }
    if constexpr (EPI == EPI_LOGITS) {
        /* the argmax partials are read by the last workgroup: stores acknowledged first */
        wait_stores();
        bar();
        if (sig && LG_TID == 0) cst(&P.progress[blockIdx.x], sig);
    } else if (sig) pk_signal(P, sig);
    stamp(tr, 3);
    if (EPI == EPI_LOGITS) {
        if (LG_TID == 0) {
            const uint32_t old = __hip_atomic_fetch_add(P.amax_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_int[0] = old == gridDim.x - 1;
        }
        bar();
        if (s_int[0]) {   /* workgroup-uniform */
            const int bi = argmax_partials<PK_THREADS>(P, gridDim.x);
            if (LG_TID == 0) {
                cst(P.tok_out, bi == 0x7fffffff ? 0 : bi);
                cst(P.amax_cnt, 0u);
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* attention phase                                                      */
/* ------------------------------------------------------------------ */
/* One head of HD values held 4 per lane (lanes 4l < HD): Qwen3 QK RMSNorm
 * (when has_norm, weights g of the lane's 4 values) and adjacent-pair RoPE
 * (fr = the frequencies of the lane's two pairs), exactly as
 * k_qk_norm_rope_kv. */
template <int HD>
__device__ __forceinline__ void norm_rope_head(float e[4], bool has_norm, float4 g, float eps, int rope_dim, int pos,
                                               float2 fr)
{
    const int lane = LG_TID & 63;
    const bool act = 4 * lane < HD;
    {
        /* computed whether or not the model has QK norms, and selected: the
         * weights' load is used unconditionally and stays where it is issued */
        float ss = act ? lg_sq4(make_float4(e[0], e[1], e[2], e[3])) : 0.0f;
        ss = lg_group_sum<64>(ss);
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
        const bool nrm = has_norm && act;
        e[0] = nrm ? e[0] * sc * g.x : e[0];
        e[1] = nrm ? e[1] * sc * g.y : e[1];
        e[2] = nrm ? e[2] * sc * g.z : e[2];
        e[3] = nrm ? e[3] * sc * g.w : e[3];
    }
    int rd = rope_dim < HD ? rope_dim : HD;
    rd &= ~1;
    if (act) {
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            const int i = 4 * lane + j;
            if (i < rd) {
                const float ang = (float)pos * (j == 0 ? fr.x : fr.y);
                float s, c;
                sincosf(ang, &s, &c);
                const float x0 = e[j], x1 = e[j + 1];
                e[j] = lg_fma2(x0, c, -x1, s);
                e[j + 1] = lg_fma2(x0, s, x1, c);
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

/* combine two online-softmax states (max m and sum l in log2 units, weighted
 * sum o); a state with m = -inf is empty */
__device__ __forceinline__ void osm_merge(float& m, float& l, float* o, float m2, float l2, const float* o2, int n)
{
    const float mn = fmaxf(m, m2);
    const float a = m == -INFINITY ? 0.0f : lg_exp2(m - mn);
    const float b = m2 == -INFINITY ? 0.0f : lg_exp2(m2 - mn);
    l = lg_fma2(l, a, l2, b);
    for (int i = 0; i < n; i++) o[i] = lg_fma2(o[i], a, o2[i], b);
    m = mn;
}

/* Attention units (NQ query heads of kv head g, chunk c of positions
 * [c*chunk, ...) <= pos), split by pk_attn_split.  A unit issues all its
 * loads at once -- its q heads, k and v of g, and every K and V slice of its
 * (at most pk_att_steps) steps, held in registers -- so it costs one memory
 * round trip (with a dependency wait, the loads follow it).  Then QK-norm +
 * RoPE of the heads into LDS, and one pass over the positions with an
 * online softmax per lane group in log2 units (LPP lanes hold one position,
 * 8 dims each); the lane groups of a wave combine by lane permutes, the
 * waves in LDS.  Output: the unit's unnormalised partial (o, and (m, l) per
 * head), merged by the consumer's build (MergeSrc); past PK_ATT_MERGE chunks
 * the last unit of each group of pk_att_group chunks (atomic counter) merges
 * the group into one of the layer's PK_ATT_MERGE group slots.  The first unit of g's last chunk also writes the fp16 cache
 * row pos. */
template <int HD, int NREP, int NQ, bool BATCHES, int WPC = 1, bool GMAJOR = false>
__device__ __forceinline__ void phase_attn(const PkParams& P, const PkLayer& L, int layer, int pos_arg,
                                           const float* __restrict__ qkv, uint64_t wait_target, uint64_t sig,
                                           uint64_t* tr, bool stamp0 = true, const uint64_t* gwords = nullptr,
                                           int gsz = 0)
{
    int pos = pos_arg;   /* FIX: first read after the unit's loads (below) */
    constexpr int HDP = pk_hdp(HD);        /* lane layout width: HD padded to a power of two */
    constexpr int LPP = HDP / 8;           /* lanes per position */
    constexpr int GLV = HD / 8;            /* lanes of a position holding values (the rest zero) */
    constexpr int PPW = 64 / LPP;          /* positions per wave step */
    constexpr int PPB = PK_WAVES * PPW;    /* positions per WG step */
    constexpr int MAXST = pk_att_steps(NREP);
    constexpr int NSUB = NREP / NQ;       /* units per (kv head, chunk) */
    constexpr int NH = (NQ + PK_WAVES) / PK_WAVES;     /* heads normed per wave: NQ q + 1 k */
    static_assert(PPB == PK_THREADS * 8 / HDP, "step geometry of pk_attn_split");
    static_assert(HD % 16 == 0 && HD <= 128, "head_dim: 48, 64, 128 (a multiple of 16 up to 128)");
    static_assert(NREP % NQ == 0, "query heads per unit divide the group");
    const int lane = LG_TID & 63, wave = LG_TID >> 6;
    const int gl = lane & (LPP - 1), grp = lane / LPP;
    const int kvd = P.kv_dim;
    /* FIX (the short-context units): fixed chunks, position-free rows */
    constexpr bool FIX = !BATCHES;
    static_assert(!FIX || NQ == 1, "short-context units hold one query head");
    /* (FIX: nch is computed after the unit's loads are issued, the first use
     * of pos) */
    int chunk, nch = 0;
    if (FIX) chunk = pk_att_fch(HD, NREP);
    else pk_attn_split(pos + 1, HD, NREP, pk_att_max_nch(P), &chunk, &nch);
    const int ngc = FIX ? 0 : P.n_kv * nch;   /* (kv head, chunk) pairs */
    const int nunits = FIX ? P.n_heads * PK_ATT_MERGE : ngc * NSUB;
    /* unit -> kv head, chunk, query-head subset */
    /* (GMAJOR, long-context units of the fused QKV + attention kernel: kv
     * head fastest, so unit u belongs to KV group u % n_kv like workgroup u) */
    auto unit_g = [&](int u) { return FIX ? u % P.n_kv : GMAJOR ? (u % ngc) % P.n_kv : (u % ngc) / nch; };
    auto unit_c = [&](int u) { return FIX ? u / P.n_heads : GMAJOR ? (u % ngc) / P.n_kv : (u % ngc) % nch; };
    auto unit_q = [&](int u) { return FIX ? (u / P.n_kv) % NREP : u / ngc; };
    const size_t loff = (size_t)layer * P.n_ctx * kvd;
    const float scale2 = 1.44269504088896341f / sqrtf((float)HD);   /* log2(e) / sqrt(head_dim) */
    float* po = P.att_po + (size_t)layer * P.att_slots * P.n_embed;
    float* pml = P.att_pml + (size_t)layer * P.att_slots * P.n_heads * 2;
    /* the group slots (past PK_ATT_MERGE chunks, chunk c merged into group
     * c / gsz by the group's last unit): written by nobody else in a launch,
     * so no cache holds a stale copy of them */
    float* po_m = po + (size_t)(P.att_slots - PK_ATT_MERGE) * P.n_embed;
    float* pml_m = pml + (size_t)(P.att_slots - PK_ATT_MERGE) * P.n_heads * 2;

    if (stamp0) stamp(tr, 0);
    /* K/V slices of the unit's steps (static indices only): one batch of
     * MAXST steps, or (BATCHES) two sets of MAXST/2 steps, the next one
     * loading while the other computes */
    /* WPC = 2: two workgroups per CU (128 VGPRs): 1 / LG_ATT_H2 of the
     * steps per set, q read from LDS */
    static_assert(WPC == 1 || (WPC == 2 && BATCHES), "two workgroups per CU: long-context units");
    constexpr int NB = BATCHES ? 2 : 1, H0 = WPC == 1 ? MAXST / NB : MAXST / NB / LG_ATT_H2;
    constexpr int H = H0 < 1 ? 1 : H0;   /* steps per register set */
    static_assert(H >= 1, "a register set holds at least one step");
    uint4 kb[NB][H], vb[NB][H];
    float4 hx[NH], hv;            /* this wave's heads h = wave + PK_WAVES*j: q (h < NQ) or k, and v */
    /* unconditional loads (see Rows): positions outside the unit and the
     * row pos itself (not in the cache yet) load the unit's first row */
    auto load_kv = [&](int set, int u, int sb) {   /* steps sb..sb+H-1 into set `set` */
        const int g = unit_g(u), c = unit_c(u);
        const int t0 = c * chunk;
#pragma unroll
        for (int st = 0; st < H; st++) {
            int t = t0 + (sb + st) * PPB + wave * PPW + grp;
            /* FIX: every row of the chunk inside the cache (rows past pos
             * are loaded and not used); else rows of the unit below pos */
            if (FIX) t = min(t, P.n_ctx - 1);
            else t = t < min(t0 + chunk, pos + 1) && t != pos ? t : t0;
            const size_t o = loff + (size_t)t * kvd + (size_t)g * HD + min(gl, GLV - 1) * 8;
            kb[set][st] = *(const uint4*)(P.kc + o);
            vb[set][st] = *(const uint4*)(P.vc + o);
        }
    };
    /* q/k norm weights (a dummy slice of the rope table when the model has
     * none) and the rope frequencies of the lane's two pairs */
    const bool has_norm = L.q_norm != nullptr;
    const int l4 = 4 * (lane % (HD / 4));
    float4 ng[NH];
    float2 fr;
    auto load_heads = [&](int u) {
        const int g = unit_g(u), q0 = g * NREP + unit_q(u) * NQ;
#pragma unroll
        for (int j = 0; j < NH; j++) {
            const int h = min(wave + PK_WAVES * j, NQ);
            const float* srcp = h < NQ ? qkv + (size_t)(q0 + h) * HD : qkv + P.n_embed + (size_t)g * HD;
            hx[j] = *(const float4*)(srcp + l4);
            const float* nwp = has_norm ? (h < NQ ? L.q_norm : L.k_norm) : P.rope_freq;
            ng[j] = *(const float4*)(nwp + l4);
        }
        hv = *(const float4*)(qkv + P.n_embed + kvd + (size_t)g * HD + l4);
        fr = *(const float2*)(P.rope_freq + l4 / 2);
    };
    const bool has = (int)blockIdx.x < nunits;
    /* with a dependency wait (the persistent kernel), the short-context
     * unit's K/V rows -- cache rows of earlier steps, position-free -- load
     * before it, by waves 1.. (wave 0 polls: its loads would hold the poll
     * back), and the heads after it */
    /* (GMAJOR: the long unit's first register set likewise -- rows of
     * earlier steps, its chunk fixed by the position known at launch) */
    const bool pre = (FIX || GMAJOR) && wait_target != 0;
    if (pre && has && wave != 0) load_kv(0, blockIdx.x, 0);
    if (wait_target) {
        if (gwords) group_wait(P, gwords, gsz, wait_target);
        else pk_wait(P, wait_target);
    }
    if (!FIX && !has) stamp(tr, 1);   /* FIX: after the loop (no store ahead of the unit's loads) */

    /* one unit: the loads, QK-norm/RoPE (+ the KV row), scores, partials */
    auto do_unit = [&](int u) {
        /* long-context units ordered (q-head subset, kv head, chunk): the
         * NSUB units that read the same K/V rows sit ngc apart, on the same
         * XCD (and L2) when ngc is a multiple of 8; short ones (kv head
         * fastest) put a kv head's query heads and chunks on one XCD when
         * n_kv is a multiple of 8 */
        const int g = unit_g(u), c = unit_c(u), qsub = unit_q(u);
        const int q0 = g * NREP + qsub * NQ;   /* first query head of the unit */
        const int t0 = c * chunk;
        load_heads(u);
        lg_issue_order();   /* heads first, then K/V */
        if (!pre || wave == 0 || u != (int)blockIdx.x) load_kv(0, u, 0);
        if (FIX) {
            /* the position from here on: an empty asm pins its first use
             * behind the loads above (it may still be in flight) */
            asm volatile("" : "+v"(pos));
            pos = __builtin_amdgcn_readfirstlane(pos);
            nch = (pos + chunk) / chunk;
        }
        if (FIX && c >= nch) {   /* a chunk past the context */
            if (u == (int)blockIdx.x) stamp(tr, 1);
            return;
        }
        const int t1 = min(t0 + chunk, pos + 1);
        const int nsteps = (t1 - t0 + PPB - 1) / PPB;
        /* v of g into LDS, by every wave (the same values): an unconditional
         * use keeps its load ahead of the K/V loads */
        *(float4*)(s_kv + HDP + l4) = hv;
        if (HD < HDP && 4 * lane >= HD && 4 * lane < HDP)
            *(float4*)(s_kv + HDP + 4 * lane) = make_float4(0.f, 0.f, 0.f, 0.f);
        /* q heads q0.., then k of g: normed/roped into LDS (waves past
         * the last head compute a copy and store nothing: the operands' loads
         * are used unconditionally and stay where they are issued) */
#pragma unroll
        for (int j = 0; j < NH; j++) {
            const int h = wave + PK_WAVES * j;
            const bool is_q = h < NQ;
            float e[4] = {hx[j].x, hx[j].y, hx[j].z, hx[j].w};
            norm_rope_head<HD>(e, has_norm, ng[j], P.eps, P.rope_dim, pos, fr);
            if (h <= NQ) {
                if (HD < HDP && 4 * lane >= HD && 4 * lane < HDP)
                    *(float4*)((is_q ? s_q + h * HDP : s_kv) + 4 * lane) = make_float4(0.f, 0.f, 0.f, 0.f);
                if (4 * lane < HD) {
                    float* dst = is_q ? s_q + h * HDP : s_kv;
                    *(float4*)(dst + 4 * lane) = make_float4(e[0], e[1], e[2], e[3]);
                    if (!is_q) {
                        if (c == nch - 1 && qsub == 0) {
                            /* fp16 KV row pos (fast/ligguf_fast_qk.cpp:57-62), read from the next token on */
                            const size_t o = loff + (size_t)pos * kvd + (size_t)g * HD + 4 * lane;
                            const uint32_t klo = (uint32_t)lg_f2h(e[0]) | ((uint32_t)lg_f2h(e[1]) << 16);
                            const uint32_t khi = (uint32_t)lg_f2h(e[2]) | ((uint32_t)lg_f2h(e[3]) << 16);
                            const uint32_t vlo = (uint32_t)lg_f2h(hv.x) | ((uint32_t)lg_f2h(hv.y) << 16);
                            const uint32_t vhi = (uint32_t)lg_f2h(hv.z) | ((uint32_t)lg_f2h(hv.w) << 16);
                            *(uint2*)(P.kc + o) = make_uint2(klo, khi);
                            *(uint2*)(P.vc + o) = make_uint2(vlo, vhi);
                        }
                    }
                }
            }
        }
        bar();
        if (u == (int)blockIdx.x) stamp(tr, 1);
        /* q in registers; with 8 query heads per KV head it is re-read from
         * LDS each step (registers go to K/V and the accumulators) */
        constexpr bool QIN = NQ <= 4 && WPC == 1;   /* q in registers */
        constexpr int QREG = QIN ? NQ : 1;
        float qr[QREG][8];
#pragma unroll
        for (int r = 0; r < QREG; r++)
#pragma unroll
            for (int i = 0; i < 8; i++) qr[r][i] = QIN ? s_q[r * HDP + gl * 8 + i] : 0.0f;

        /* one pass: scores, online softmax, p.V (t == pos uses the fp32 k/v
         * of this step, fast/ligguf_fast_qk.cpp:77-79,98-99) */
        float m[NQ], l[NQ], o[NQ][8];
#pragma unroll
        for (int r = 0; r < NQ; r++) {
            m[r] = -INFINITY;
            l[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) o[r][i] = 0.0f;
        }
        /* the steps of set `set` from step sb on, in step order */
        auto process = [&](int set, int sb) {
#pragma unroll
            for (int st = 0; st < H; st++) {
                const int t = t0 + (sb + st) * PPB + wave * PPW + grp;
                if (sb + st < nsteps && t < t1) {
                    float kf[8], vf[8];
                    if (t != pos) {
                        h8(kb[set][st], kf);
                        h8(vb[set][st], vf);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; i++) { kf[i] = s_kv[gl * 8 + i]; vf[i] = s_kv[HDP + gl * 8 + i]; }
                    }
                    /* the heads' scores, then their lane-group sums step by
                     * step across the heads (independent permutes back to
                     * back, no wait states between them) */
                    float sc[NQ];
#pragma unroll
                    for (int r = 0; r < NQ; r++) {
                        float qv[8];
#pragma unroll
                        for (int i = 0; i < 8; i++) qv[i] = QIN ? qr[r < QREG ? r : 0][i] : s_q[r * HDP + gl * 8 + i];
                        sc[r] = 0.0f;
#pragma unroll
                        for (int i = 0; i < 8; i++) sc[r] += qv[i] * kf[i];
                    }
                    lg_group_sum_n<LPP, NQ>(sc);
                    /* online softmax with a lazily moved reference: the sums
                     * are kept relative to m, which moves (and rescales
                     * them) only when a score passes m + PK_ATT_LAZY -- each
                     * weight 2^(s - m) stays below 2^PK_ATT_LAZY, and the
                     * state (m, l, o) stands for sum 2^(s - m) as before */
#pragma unroll
                    for (int r = 0; r < NQ; r++) {
                        const float s2 = sc[r] * scale2;
                        const bool up = s2 > m[r] + PK_ATT_LAZY;   /* also while m = -inf */
                        if (__builtin_amdgcn_ballot_w64(up)) {     /* wave-uniform, rare past the first rows */
                            const float mn = up ? s2 : m[r];
                            const float a = up ? lg_exp2(m[r] - mn) : 1.0f;   /* 0 while m = -inf */
                            l[r] *= a;
#pragma unroll
                            for (int i = 0; i < 8; i++) o[r][i] *= a;
                            m[r] = mn;
                        }
                        const float pw = lg_exp2(s2 - m[r]);
                        l[r] += pw;
#pragma unroll
                        for (int i = 0; i < 8; i++) o[r][i] = __builtin_fmaf(pw, vf[i], o[r][i]);
                    }
                }
            }
        };
        if (!BATCHES) {
            process(0, 0);   /* one batch: chunks of <= MAXST steps */
        } else {
            /* half-batches alternate between the two sets; the set not being
             * computed loads (past the last step: clamped rows, unused) */
            for (int sb = 0; sb < nsteps; sb += 2 * H) {
                load_kv(NB - 1, u, sb + H);
                process(0, sb);
                if (sb + H >= nsteps) break;
                load_kv(0, u, sb + 2 * H);
                process(NB - 1, sb + H);
            }
        }
        /* combine the position groups of the wave into group 0 (8-lane
         * groups first pairwise by xor 8; then 16-lane rows: row 1 -> 0 and
         * 3 -> 2, then 2 -> 0, by lane permutes), then the waves (LDS) */
        static_assert(LPP == 16 || LPP == 8, "position groups of 8 or 16 lanes");
        if constexpr (LPP == 8) {
#pragma unroll
            for (int r = 0; r < NQ; r++) {
                float o2[8];
#pragma unroll
                for (int i = 0; i < 8; i++) o2[i] = __shfl_xor(o[r][i], 8);
                const float m2 = __shfl_xor(m[r], 8), l2 = __shfl_xor(l[r], 8);
                osm_merge(m[r], l[r], o[r], m2, l2, o2, 8);
            }
        }
#pragma unroll
        for (int step = 0; step < 2; step++) {
#pragma unroll
            for (int r = 0; r < NQ; r++) {
                float o2[8];
#pragma unroll
                for (int i = 0; i < 8; i++) o2[i] = step ? lg_from_half_above(o[r][i]) : lg_from_row_above(o[r][i]);
                const float m2 = step ? lg_from_half_above(m[r]) : lg_from_row_above(m[r]);
                const float l2 = step ? lg_from_half_above(l[r]) : lg_from_row_above(l[r]);
                osm_merge(m[r], l[r], o[r], m2, l2, o2, 8);
            }
        }
        if (grp == 0) {
#pragma unroll
            for (int r = 0; r < NQ; r++) {
                if (gl < GLV) {
#pragma unroll
                    for (int i = 0; i < 8; i++) s_o[(wave * NQ + r) * HD + gl * 8 + i] = o[r][i];
                }
                if (gl == 0) { s_m[wave * NQ + r] = m[r]; s_sc[wave * NQ + r] = l[r]; }
            }
        }
        bar();
        for (int i = LG_TID; i < NQ * HD; i += PK_THREADS) {
            const int r = i / HD, d = i % HD, q = q0 + r;
            float M = -INFINITY;
            for (int w = 0; w < PK_WAVES; w++) M = fmaxf(M, s_m[w * NQ + r]);
            float O = 0.0f, Ls = 0.0f;
            for (int w = 0; w < PK_WAVES; w++) {
                const float mw = s_m[w * NQ + r];
                const float wt = mw == -INFINITY ? 0.0f : lg_exp2(mw - M);
                O += s_o[(w * NQ + r) * HD + d] * wt;
                Ls += s_sc[w * NQ + r] * wt;
            }
            cst(&po[(size_t)c * P.n_embed + (size_t)q * HD + d], O);
            if (d == 0) {
                cst(&pml[((size_t)c * P.n_heads + q) * 2], M);
                cst(&pml[((size_t)c * P.n_heads + q) * 2 + 1], Ls);
            }
        }
        if (nch > PK_ATT_MERGE) {
            /* chunk c belongs to group c / gsz (at most PK_ATT_MERGE groups):
             * the group's last unit (atomic counter per heads and group)
             * merges its chunks into the group slot as one partial (o, m, l);
             * the att_out build merges the groups */
            const int gsz = pk_att_group(nch), G = c / gsz;
            const int c_lo = G * gsz, cnt = min(gsz, nch - c_lo);
            uint32_t* ctr = &P.attn_cnt[(g * NSUB + qsub) * PK_ATT_MERGE + G];
            wait_stores();
            bar();
            if (LG_TID == 0) {
                const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_int[0] = old == (uint32_t)(cnt - 1);
            }
            bar();
            if (s_int[0]) {
                /* weights through LDS, then each thread one output value
                 * over the group's chunks, 8 loads in flight (the
                 * consumer's formula, without the division) */
                float* s_ml = s_sc;                                   /* [cnt][NQ][2] */
                float* s_w = s_sc + PK_ATT_MAX_NCH * 2 * PK_MAX_NREP; /* [cnt][NQ] */
                for (int i = LG_TID; i < cnt * NQ; i += PK_THREADS) {
                    const float2 v = cld2(&pml[((size_t)(c_lo + i / NQ) * P.n_heads + q0 + i % NQ) * 2]);
                    s_ml[2 * i] = v.x;
                    s_ml[2 * i + 1] = v.y;
                }
                bar();
                if (LG_TID < NQ) {
                    const int r = LG_TID;
                    float M = -INFINITY;
                    for (int cc = 0; cc < cnt; cc++) M = fmaxf(M, s_ml[(cc * NQ + r) * 2]);
                    float Ls = 0.0f;
                    for (int cc = 0; cc < cnt; cc++) {
                        const float wgt = lg_exp2(s_ml[(cc * NQ + r) * 2] - M);
                        s_w[cc * NQ + r] = wgt;
                        Ls += s_ml[(cc * NQ + r) * 2 + 1] * wgt;
                    }
                    cst(&pml_m[((size_t)G * P.n_heads + q0 + r) * 2], M);
                    cst(&pml_m[((size_t)G * P.n_heads + q0 + r) * 2 + 1], Ls);
                }
                bar();
                for (int i = LG_TID; i < NQ * HD; i += PK_THREADS) {
                    const int r = i / HD;
                    const float* col = po + (size_t)c_lo * P.n_embed + (size_t)q0 * HD + i;
                    float acc = 0.0f;
                    for (int c0 = 0; c0 < cnt; c0 += 8) {
                        float v[8];
#pragma unroll
                        for (int k = 0; k < 8; k++) v[k] = cld(col + (size_t)min(c0 + k, cnt - 1) * P.n_embed);
#pragma unroll
                        for (int k = 0; k < 8; k++)
                            if (c0 + k < cnt) acc += v[k] * s_w[(c0 + k) * NQ + r];
                    }
                    cst(&po_m[(size_t)G * P.n_embed + (size_t)q0 * HD + i], acc);
                }
                if (LG_TID == 0) cst(ctr, 0u);
            }
        }
        bar();
    };
    if (FIX) {
        /* at most one unit per workgroup (pk_att_long): no loop, so no
         * wait at a loop head for loads of a previous iteration */
        if (has) do_unit((int)blockIdx.x);
    } else {
        for (int u = blockIdx.x; u < nunits; u += gridDim.x) do_unit(u);
    }
    if (FIX && !has) stamp(tr, 1);
    stamp(tr, 2);
    if (sig) pk_signal(P, sig);
    stamp(tr, 3);
}

/* the attention phase with the units pk_att_long picks for this context
 * (both bodies inlined; the choice is uniform over the grid) */
template <int HD, int NREP>
__device__ __forceinline__ void phase_attn_any(const PkParams& P, const PkLayer& L, int layer, int pos,
                                               const float* __restrict__ qkv, uint64_t wait_target, uint64_t sig,
                                               uint64_t* tr)
{
    if (!pk_att_long(pos, HD, NREP, P.n_kv, gridDim.x))
        phase_attn<HD, NREP, 1, false>(P, L, layer, pos, qkv, wait_target, sig, tr);
    else
        phase_attn<HD, NREP, NREP, true>(P, L, layer, pos, qkv, wait_target, sig, tr);
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

/* items per batch (B) and batches held at once (R, phase_mv's ring) of each
 * matvec phase, shared by the fused and the persistent kernels; LT/NE/NF are
 * the layer type and its slots per lane at n_embed / n_ff, OT/NO the output
 * head's */
#ifndef LG_QKV_B
#define LG_QKV_B (Batch<LT, NE, 1, 2, 512>::value)
#endif
#ifndef LG_QKV_R
/* a second batch in flight while a batch takes at most 128 bytes a lane
 * (all but F32 rows) */
#define LG_QKV_R (Batch<LT, NE, 1, 2, 512>::bytes > 128 ? 1 : 2)
#endif
#ifndef LG_AO_B
#define LG_AO_B (Batch<LT, NE, 1, 1, 512>::value)
#endif
#ifndef LG_AO_R
#define LG_AO_R 2
#endif
#ifndef LG_UG_B
#define LG_UG_B 1
#endif
#ifndef LG_UG_R
#define LG_UG_R (Batch<LT, NE, 2, 1, 512>::bytes > 256 ? 1 : 2)
#endif
#ifndef LG_DN_B
#define LG_DN_B (Batch<LT, NF, 1, 1, 512>::value)
#endif
#ifndef LG_DN_R
/* a second batch in flight only while the rows of one fit the register budget
 * (Q5_K / Q6_K down rows of 14336 values spilled with two) */
#define LG_DN_R (Batch<LT, NF, 1, 1, 512>::bytes > 192 ? 1 : 2)
#endif
#ifndef LG_OUT_B
#define LG_OUT_B 1
#endif
#ifndef LG_OUT_R
#define LG_OUT_R 2
#endif

/* slots per lane at width n_embed = 4096: one 64-value slot, two Q8_0 slots */
template <int T>
struct NsE {
    static constexpr int value = T == LG_Q8_0 ? 2 : 1;
};

