/* lg_fused.hip -- the per-token step of inference()
 * (fast/ligguf_fast_qk.cpp:24-144) as fused kernels -- by default three per
 * layer (qkv + attn + ao in k_f_qkva, the ao rows split by KV group; ug;
 * down) -- plus one for the output head, meant to be replayed from a HIP
 * graph.
 *
 * The phases of layer l (one workgroup of 8 waves per CU in every kernel):
 *   qkv   rmsnorm(x)->Q8 in LDS (every workgroup), Q|K|V rows      -> qkv[l]
 *   attn  QK-norm + RoPE + fp16 KV write of row pos, one-pass online
 *         softmax over (kv head, chunk) units               -> partials
 *   ao    merge of the partials, Q8(att) in LDS, att_out rows
 *         + residual                                              -> xm[l]
 *   ug    rmsnorm(xm)->Q8, up|gate row pairs + SwiGLU             -> hb[l]
 *   down  Q8(hb) in LDS, down rows + residual                     -> xs[l+1]
 * then out: rmsnorm -> output rows -> logits, per-WG argmax, the last
 * workgroup reduces it (sampler_greedy, fast/ligguf_fast_qk.cpp:146-160) and
 * advances the device step record to {token, pos + 1}.
 *
 * The parameter block and the layer's weights are kernel arguments (by
 * value): pointers read from them are known to be global, so every access
 * is a global_load/store -- a
 * flat access would also count against lgkmcnt, and each LDS wait of a
 * build would then wait for all of the wave's outstanding weight loads.
 * Every kernel issues its weight loads first and builds its activation
 * while they are in flight; the kernel boundary is the only grid-wide sync
 * (a graph replays 3*n_layers + 1 kernels at ~1.6 us of fixed cost each,
 * cheaper than a flag sync through memory), the KV groups' barriers inside
 * k_f_qkva stay within one XCD each.  The token and position come from device
 * memory (PkStep), so one captured graph serves every step.  The phase code
 * is the persistent kernel's (lg_phase.h): same arithmetic, same bits.
 */
#include "lg_phase.h"

/* output-head workgroups per CU: the head's rows need no more than one
 * build per workgroup, and more workgroups hold more rows in flight */
#ifndef LG_OUT_WGS
#define LG_OUT_WGS 1
#endif
static_assert(LG_OUT_WGS >= 1 && LG_OUT_WGS <= LG_OUT_MAX_WGS, "argmax partials");

/* trace slot of phase k of layer l for this workgroup (PkStep.trace, one
 * slot per workgroup of an nwg-workgroup layer grid) */
__device__ __forceinline__ uint64_t* f_tr_n(const PkStep* Sd, int l, int k, int nwg)
{
    uint64_t* t = Sd->trace;
    return t ? t + ((size_t)(5 * l + k) * nwg + blockIdx.x) * 4 : nullptr;
}
__device__ __forceinline__ uint64_t* f_tr(const PkStep* Sd, int l, int k) { return f_tr_n(Sd, l, k, gridDim.x); }

/* activation trace slot k (a kernel argument: NULL in the captured graph,
 * so a traced step is launched directly) */
__device__ __forceinline__ uint8_t* f_atr(uint8_t* atr, const PkParams& P, int k)
{
    return atr ? atr + (size_t)k * P.act_stride : nullptr;
}

/* Widths.  S carries the slots per lane of a row of n_embed values (NE for
 * the layer type, NO for the output type) and of n_ff values (NF), and the
 * 256-value activation chunks per wave of an n_embed (CE) and an n_ff (CF)
 * wide build; the widths themselves are runtime values (phase_mv masks the
 * slots and chunks past them). */
template <int NE_, int NO_, int CE_, int NF_, int CF_>
struct FShape {
    static constexpr int NE = NE_, NO = NO_, CE = CE_, NF = NF_, CF = CF_;
};

/* EMB: layer 0, whose input is the embedding row of the step's token */
template <int LT, class S, bool EMB>
__global__ __launch_bounds__(PK_THREADS) void k_f_qkv(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd,
                                                      int l, uint8_t* atr)
{
    constexpr int NE = S::NE;
    const int ne = P.n_embed, qs = ne + 2 * P.kv_dim;
    float* xin = P.xs + (size_t)l * ne;
    const int pos = Sd->pos;
    const int tok = pos < Sd->feed_end ? P.feed[pos] : Sd->tok;
    phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, EMB ? BLD_EMB : BLD_RMS, S::CE, LG_QKV_R>(
        P, tok, L.qkv, L.qkv_rsz, qs, 0, L.att_norm, xin, nullptr, P.qkv + (size_t)l * qs, xin, 0, 0,
        f_tr(Sd, l, 0), f_atr(atr, P, 4 * l), ne);
}

/* Q|K and V of different types (L.v): one rmsnorm build, the Q|K rows,
 * then the V rows on the activation the first sweep left in LDS, mapped to
 * start on the waves the Q|K rows left with fewer items */
template <int LT, int VT, class S, bool EMB>
__global__ __launch_bounds__(PK_THREADS) void k_f_qkv2(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd,
                                                       int l, uint8_t* atr)
{
    constexpr int NE = S::NE;
    const int ne = P.n_embed, kvd = P.kv_dim, qs = ne + 2 * kvd;
    float* xin = P.xs + (size_t)l * ne;
    float* out = P.qkv + (size_t)l * qs;
    const int pos = Sd->pos;
    const int tok = pos < Sd->feed_end ? P.feed[pos] : Sd->tok;
    phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, EMB ? BLD_EMB : BLD_RMS, S::CE, LG_QKV_R>(
        P, tok, L.qkv, L.qkv_rsz, ne + kvd, 0, L.att_norm, xin, nullptr, out, xin, 0, 0, f_tr(Sd, l, 0),
        f_atr(atr, P, 4 * l), ne);
    const int nwv = gridDim.x * PK_WAVES, left = (ne + kvd) % nwv;
    phase_mv<VT, NE, (Batch<VT, NE, 1, 2, 512>::value), 1, EPI_STORE, BLD_KEEP, S::CE, LG_QKV_R>(
        P, tok, L.v, L.v_rsz, kvd, 0, nullptr, nullptr, nullptr, out + ne + kvd, nullptr, 0, 0, nullptr, nullptr, ne,
        MergeSrc{nullptr, nullptr, 0, 0}, left ? nwv - left : 0);
}

/* att_out rows of this workgroup, KV group g's share of each (the fused
 * QKV + attention + att_out kernel, after the group's attention units).
 * The group's query heads are values 512g .. 512g+511 of the attention
 * vector -- two Q8_K blocks (or 16 Q8_0 blocks) of their own, quantized by
 * the group alone -- and slots 8g .. 8g+7 of every 4096-value att_out row.
 * After a second group barrier (every unit of the group stored its
 * partials), waves 0 and 1 merge the group's two 256-value chunks as the
 * att_out build does (MergeAct, chunks in ascending order) and quantize
 * them into s_act; then lane 8q + j of each wave dots slot 8g + j of row q of a pass
 * and the 8-lane sum -- the first three steps of lg_wave_sum -- is the
 * row's group partial, stored to P.ao_part[g][row].  The next up|gate
 * build adds the 8 partials in lg_wave_sum's order (PartSum), so xm is the
 * att_out phase's bit for bit.  Rows of workgroup r: r * rpw .. (rpw =
 * n_embed / group size, at most 64 * AO_NP), pass p of wave w rows
 * 64p + 8w + q of them.  Waves 1.. issue their row loads before the
 * barrier wait (wave 1's merge loads go behind them); wave 0 polls, then
 * issues the merge loads and its rows. */
#define AO_NP 2
template <int LT, int HD, int NREP>
__device__ __forceinline__ void phase_ao_group(const PkParams& P, const PkLayer& L, int l, int pos, int g, int r,
                                               int gsz, const uint64_t* words, uint64_t* mine, uint64_t round2,
                                               uint8_t* atr, uint64_t* tr)
{
    using F = Fmt<LT>;
    constexpr int QT = lg_act_qt(LT);
    static_assert(F::VALS == 64 && NREP * HD == 8 * 64, "a group's slice is 8 slots of 64 values");
    const int lane = LG_TID & 63, wave = __builtin_amdgcn_readfirstlane(LG_TID >> 6);
    const int ne = P.n_embed, rpw = ne / gsz, r0 = r * rpw;
    const int j = lane & 7, q = lane >> 3, slot = 8 * g + j;
    stamp(tr, 0);
    typename F::W w[AO_NP];
    auto load_rows = [&]() {
#pragma unroll
        for (int p = 0; p < AO_NP; p++) {
            const int i = r0 + min(64 * p + 8 * wave + q, rpw - 1);
            F::load_w(w[p], L.ao + (size_t)i * L.ao_rsz, slot);
        }
    };
    /* this workgroup's attention partials are stored (and acknowledged by
     * group_arrive) before its rows load: the acknowledgement wait would
     * wait for the row loads too */
    group_arrive(mine, round2);
    if (wave != 0) load_rows();
    group_wait(P, words, gsz, round2);
    stamp(tr, 1);
    if (wave < 2) {   /* wave w: chunk 2g + w */
        const MergeSrc ms = att_partials<HD, NREP>(P, l, pos);
        MergeAct<1> m0;
        m0.load_at(ms, P.n_heads, ne, (2 * g + wave) * 256 + 4 * lane);
        lg_issue_order();
        if (wave == 0) load_rows();
        ActSrc<1> a0;
        m0.merge(ms.nch, a0);
        const float v0[4] = {a0.v[0].x, a0.v[0].y, a0.v[0].z, a0.v[0].w};
        lg_emit(v0, QT, s_act, 2 * g + wave, 256);
    }
    bar();
    stamp(tr, 2);
    if (atr && r == 0) {
        /* activation trace (tests): the group's two chunks as built */
        constexpr int CB = QT == LG_Q8_K ? LG_BS_Q8_K : 8 * LG_BS_Q8_0;
        uint32_t* dst = (uint32_t*)(atr + (size_t)(2 * g) * CB);
        const uint32_t* src = (const uint32_t*)(s_act + (size_t)(2 * g) * CB);
        for (int i = LG_TID; i < 2 * CB / 4; i += PK_THREADS) dst[i] = src[i];
    }
    typename F::Act act;
    F::load_act(act, s_act, slot);
    float pv[AO_NP];
#pragma unroll
    for (int p = 0; p < AO_NP; p++) {
        float a = 0.0f;
        a += F::dot(w[p], act, slot);
        pv[p] = lg_group_sum<8>(a);
    }
    /* lanes 8p + q gather row q of pass p: one store of 8 consecutive
     * values per pass */
    float* out = P.ao_part + (size_t)g * ne;
#pragma unroll
    for (int p = 0; p < AO_NP; p++) {
        const float v = __shfl(pv[p], 8 * (lane & 7), 64);
        const int li = 64 * p + 8 * wave + (lane & 7);
        if ((lane >> 3) == p && li < rpw) out[r0 + li] = v;
    }
    stamp(tr, 3);
}

/* Q|K|V rows and the short-context attention units of one KV group in one
 * kernel.  Workgroup b works for KV group g = b % n_kv: first the group's
 * rows -- q of its NREP heads, k and v of head g -- split over the group's
 * nwg / n_kv workgroups (the V rows from L.v when VT is not 0, on the
 * activation the Q|K sweep left in LDS), then, once every workgroup of the
 * group has stored its rows (group_arrive / group_wait), attention unit b,
 * which belongs to group g by the units' order (kv head fastest): a
 * short-context unit (one query head, a fixed chunk) or (LONG) a
 * long-context one (the group's query heads, chunk b / n_kv of
 * pk_attn_split's).  The unit's K/V cache rows (its first register set)
 * load before the wait.  With the workgroups of a
 * group on one XCD (workgroup b on XCD b % 8, n_kv = 8) the barrier stays in
 * that XCD's L2.  The same rows, units and arithmetic as k_f_qkv(2) +
 * k_f_attn, so the same bits. */
template <int LT, int VT, class S, int HD, int NREP, bool EMB, bool LONG, bool AO = false>
__global__ __launch_bounds__(PK_THREADS) void k_f_qkva(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd,
                                                       int l, uint8_t* atr)
{
    constexpr int NE = S::NE;
    const int ne = P.n_embed, kvd = P.kv_dim, qs = ne + 2 * kvd;
    const int nkv = P.n_kv, g = (int)blockIdx.x % nkv, gsz = (int)gridDim.x / nkv, r = (int)blockIdx.x / nkv;
    float* xin = P.xs + (size_t)l * ne;
    float* out = P.qkv + (size_t)l * qs;
    uint64_t* words = P.grp_cnt + (size_t)g * gsz;   /* the group's words, this workgroup's at r */
    const uint64_t round = group_round(words + r);
    const int pos = Sd->pos;
    const int tok = pos < Sd->feed_end ? P.feed[pos] : Sd->tok;
    const WaveSet ws{r * PK_WAVES, gsz * PK_WAVES};
    const MergeSrc none{nullptr, nullptr, 0, 0};
    if constexpr (VT == 0) {
        const RowMap rm{NREP * HD, g * NREP * HD, HD, ne + g * HD, ne + kvd + g * HD};
        phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, EMB ? BLD_EMB : BLD_RMS, S::CE, LG_QKV_R>(
            P, tok, L.qkv, L.qkv_rsz, (NREP + 2) * HD, 0, L.att_norm, xin, nullptr, out, xin, 0, 0, f_tr(Sd, l, 0),
            f_atr(atr, P, 4 * l), ne, none, 0, rm, ws);
    } else {
        const RowMap rm{NREP * HD, g * NREP * HD, HD, ne + g * HD, 0};
        phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, EMB ? BLD_EMB : BLD_RMS, S::CE, LG_QKV_R>(
            P, tok, L.qkv, L.qkv_rsz, (NREP + 1) * HD, 0, L.att_norm, xin, nullptr, out, xin, 0, 0, f_tr(Sd, l, 0),
            f_atr(atr, P, 4 * l), ne, none, 0, rm, ws);
        const int left = ((NREP + 1) * HD) % ws.nwv;
        const RowMap rv{HD, g * HD, 0, 0, 0};
        phase_mv<VT, NE, (Batch<VT, NE, 1, 2, 512>::value), 1, EPI_STORE, BLD_KEEP, S::CE, LG_QKV_R>(
            P, tok, L.v, L.v_rsz, HD, 0, nullptr, nullptr, nullptr, out + ne + kvd, nullptr, 0, 0, nullptr, nullptr, ne,
            none, left ? ws.nwv - left : 0, rv, ws);
    }
    group_arrive(words + r, round);
    uint64_t* tr = f_tr(Sd, l, 1);
    stamp(tr, 0);
    if constexpr (LONG) phase_attn<HD, NREP, NREP, true, 1, true>(P, L, l, pos, out, round, 0, tr, false, words, gsz);
    else phase_attn<HD, NREP, 1, false>(P, L, l, pos, out, round, 0, tr, false, words, gsz);
    if constexpr (AO)
        phase_ao_group<LT, HD, NREP>(P, L, l, pos, g, r, gsz, words, words + r, round + 1, f_atr(atr, P, 4 * l + 1),
                                     f_tr(Sd, l, 2));
}

/* LONG: the long-context units (the host picks by pk_att_long of the step's
 * position); otherwise one-head single-batch units.  Two kernels, so the
 * short-context one carries no long-context code or registers. */
template <int HD, int NREP, bool LONG>
__global__ __launch_bounds__(PK_THREADS) __attribute__((amdgpu_waves_per_eu(LONG ? 2 * LG_ATT_WGS : 2)))
void k_f_attn(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd, int l)
{
    const int ne = P.n_embed, qs = ne + 2 * P.kv_dim;
    if constexpr (LONG) {
        /* a grid of P.att_grid workgroups, LG_ATT_WGS per CU; the step trace
         * holds the first gridDim.x / LG_ATT_WGS */
        uint64_t* tr = (int)blockIdx.x < (int)gridDim.x / LG_ATT_WGS
                           ? f_tr_n(Sd, l, 1, gridDim.x / LG_ATT_WGS) : nullptr;
        phase_attn<HD, NREP, NREP, true, LG_ATT_WGS>(P, L, l, Sd->pos, P.qkv + (size_t)l * qs, 0, 0, tr);
    } else {
        /* the position through a vector load issued first (its index made
         * opaque, so the compiler keeps it per lane instead of moving it to
         * a scalar register at once): the short units' loads do not depend
         * on it and go out behind it; phase_attn waits for it after them.
         * A scalar load would be waited for (lgkmcnt) with the kernel
         * arguments, before any of them. */
        uint64_t* tr = f_tr(Sd, l, 1);
        stamp(tr, 0);   /* before the position load: a later wait for the stamp's store would wait for it too */
        int z;
        asm volatile("v_mov_b32 %0, 0" : "=v"(z));
        const int pos = cld(&Sd->pos + z);
        lg_issue_order();
        phase_attn<HD, NREP, 1, false>(P, L, l, pos, P.qkv + (size_t)l * qs, 0, 0, tr, false);
    }
}

template <int LT, class S, int HD, int NREP>
__global__ __launch_bounds__(PK_THREADS) void k_f_ao(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd, int l,
                                                     uint8_t* atr)
{
    constexpr int NE = S::NE;
    const int ne = P.n_embed;
    phase_mv<LT, NE, LG_AO_B, 1, EPI_RESID, BLD_MERGE, S::CE, LG_AO_R>(
        P, 0, L.ao, L.ao_rsz, ne, 0, nullptr, nullptr, P.xs + (size_t)l * ne, P.xm + (size_t)l * ne, nullptr, 0, 0,
        f_tr(Sd, l, 2), f_atr(atr, P, 4 * l + 1), ne, att_partials<HD, NREP>(P, l, Sd->pos));
}

/* RSUM: the input is x_l + the att_out group partials (k_f_qkva<..., AO>),
 * stored by workgroup 0 as xm_l; its build loads 8 more vectors, so LG_UGS_R
 * batches of rows (a deeper ring) are in flight while it runs */
#ifndef LG_UGS_R
#define LG_UGS_R 2
#endif
template <int LT, class S, bool RSUM = false>
__global__ __launch_bounds__(PK_THREADS) void k_f_ug(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd, int l,
                                                     uint8_t* atr)
{
    constexpr int NE = S::NE;
    const int ne = P.n_embed, nff = P.n_ff;
    phase_mv<LT, NE, LG_UG_B, 2, EPI_SWIGLU, RSUM ? BLD_RSUM : BLD_RMS, S::CE, RSUM ? LG_UGS_R : LG_UG_R>(
        P, 0, L.ug, L.ug_rsz, nff, nff, L.ffn_norm, RSUM ? P.xs + (size_t)l * ne : P.xm + (size_t)l * ne, nullptr,
        P.hb + (size_t)l * nff, RSUM ? P.xm + (size_t)l * ne : nullptr, 0, 0, f_tr(Sd, l, 3), f_atr(atr, P, 4 * l + 2),
        ne);
}

template <int LT, class S>
__global__ __launch_bounds__(PK_THREADS) void k_f_down(const PkParams P, const PkLayer L, const PkStep* __restrict__ Sd, int l,
                                                       uint8_t* atr)
{
    constexpr int NF = S::NF;
    const int ne = P.n_embed, nff = P.n_ff;
    phase_mv<LT, NF, LG_DN_B, 1, EPI_RESID, BLD_PLAIN, S::CF, LG_DN_R>(
        P, 0, L.down, L.down_rsz, ne, 0, nullptr, P.hb + (size_t)l * nff, P.xm + (size_t)l * ne,
        P.xs + (size_t)(l + 1) * ne, nullptr, 0, 0, f_tr(Sd, l, 4), f_atr(atr, P, 4 * l + 3), nff);
}

/* the regrouped forms (lg_repack_rows): a head of one of them is read from
 * its copy in P.out_wr */
static constexpr bool f_is_rep(int t)
{
    return t == LG_Q8_0_R || t == LG_Q6_K_R || t == LG_Q1_G_R || t == LG_Q3_K_R || t == LG_Q1_0_R;
}

/* OT may be a regrouped form: the head's copy in P.out_wr */
template <int OT, class S>
__global__ __launch_bounds__(PK_THREADS) void k_f_out(const PkParams P, PkStep* __restrict__ Sd, uint8_t* atr)
{
    constexpr int NO = S::NO;
    const uint8_t* W = f_is_rep(OT) ? P.out_wr : P.out_w;
    const int pos = Sd->pos;
    /* the step trace holds one slot per workgroup of the layer grid: the
     * first gridDim.x / LG_OUT_WGS workgroups stamp theirs */
    const int nwg = gridDim.x / LG_OUT_WGS;
    uint64_t* tr = Sd->trace && (int)blockIdx.x < nwg
                       ? Sd->trace + ((size_t)5 * P.n_layers * nwg + blockIdx.x) * 4 : nullptr;
    phase_mv<OT, NO, LG_OUT_B, 1, EPI_LOGITS, BLD_RMS, S::CE, LG_OUT_R>(
        P, 0, W, P.out_rsz, P.vocab, 0, P.out_norm, P.xs + (size_t)P.n_layers * P.n_embed, nullptr, P.logits,
        nullptr, 0, 0, tr, f_atr(atr, P, 4 * P.n_layers), P.n_embed);
    /* s_int[0]: this workgroup reduced the argmax and wrote tok_out */
    if (s_int[0] && threadIdx.x == 0) {
        const int t = cld(P.tok_out);
        P.tok_hist[pos] = t;
        Sd->tok = t;
        Sd->pos = pos + 1;
        Sd->trace = nullptr;    /* a trace covers one step */
    }
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */
typedef void (*fused_enqueue_t)(const PkParams&, const PkLayer*, PkStep*, int, int, bool, hipStream_t, uint8_t*);

/* the regrouped form of an output type (P.out_wr), or the type itself */
static constexpr int f_rep(int t)
{
    return t == LG_Q8_0 ? LG_Q8_0_R : t == LG_Q6_K ? LG_Q6_K_R : t == LG_Q1_G ? LG_Q1_G_R : t == LG_Q3_K ? LG_Q3_K_R
         : t == LG_Q1_0 ? LG_Q1_0_R : t;
}

template <int OT, class SH>
static void f_launch_out(const PkParams& P, PkStep* S, int nwg, dim3 b, hipStream_t st, uint8_t* atr)
{
    static_assert(f_rep(OT) == OT || f_is_rep(f_rep(OT)), "k_f_out reads every form f_rep makes from P.out_wr");
    if (f_rep(OT) != OT && P.out_wr)
        hipLaunchKernelGGL((k_f_out<f_rep(OT), SH>), dim3(nwg * LG_OUT_WGS), b, 0, st, P, S, atr);
    else hipLaunchKernelGGL((k_f_out<OT, SH>), dim3(nwg * LG_OUT_WGS), b, 0, st, P, S, atr);
}

/* the V and down types a layer of type LT may carry besides LT itself */
template <int LT>
static constexpr bool f_mixable() { return LT == LG_Q4_K || LT == LG_Q5_K; }

#if LG_FUSED_PART == 0
bool lg_fused_side_type(int lt, int t)
{
    return t == lt || ((lt == LG_Q4_K || lt == LG_Q5_K) && (t == LG_Q5_K || t == LG_Q6_K));
}
#endif

/* phase 0 of layer l: Q|K|V stacked, or Q|K and a V of its own type */
template <int LT, class SH>
static void f_launch_qkv(const PkParams& P, const PkLayer& L, PkStep* S, int l, dim3 g, dim3 b, hipStream_t st,
                         uint8_t* atr)
{
    if constexpr (f_mixable<LT>()) {
        if (L.v) {
#define QKV2(VT)                                                                                                \
    do {                                                                                                        \
        if (l == 0) hipLaunchKernelGGL((k_f_qkv2<LT, VT, SH, true>), g, b, 0, st, P, L, S, l, atr);            \
        else hipLaunchKernelGGL((k_f_qkv2<LT, VT, SH, false>), g, b, 0, st, P, L, S, l, atr);                   \
    } while (0)
            if (L.v_t == LG_Q6_K_R) QKV2(LG_Q6_K_R);
            else if (L.v_t == LG_Q6_K) QKV2(LG_Q6_K);
            else if (L.v_t == LG_Q5_K) QKV2(LG_Q5_K);
            else QKV2(LT);
#undef QKV2
            return;
        }
    }
    if (l == 0) hipLaunchKernelGGL((k_f_qkv<LT, SH, true>), g, b, 0, st, P, L, S, l, atr);
    else hipLaunchKernelGGL((k_f_qkv<LT, SH, false>), g, b, 0, st, P, L, S, l, atr);
}

/* the fused QKV + attention kernel serves the step: short-context units,
 * the grid split evenly over the KV groups */
static bool f_qkva_ok(const PkParams& P, int nwg, bool long_ctx)
{
    /* long contexts: at most one unit per workgroup (pk_att_max_nch) */
    return P.qkva && nwg % P.n_kv == 0 && nwg <= LG_MAX_GROUP_WORDS && (!long_ctx || P.att_grid <= nwg);
}

/* att_out in the QKV + attention kernel, split by KV group: 8 KV groups
 * of 512 query values (8 slots of a 4096-value row of a 64-value-slot
 * format, one slot per lane), at most 64 * AO_NP rows per workgroup; the
 * long-context units' chunk groups are merged into their slots before the
 * group barrier, so the group merge reads those as the att_out build does */
template <int LT, class SH, int HD, int NREP>
static bool f_qkvao_ok(const PkParams& P, int nwg, bool long_ctx)
{
    if constexpr (Fmt<LT>::VALS != 64 || NREP * HD != 512 || SH::NE != 1) return false;
    else {
        if (!P.qkvao || !P.ao_part || !f_qkva_ok(P, nwg, long_ctx) || P.n_kv != 8 || P.n_embed != 4096)
            return false;
        const int gsz = nwg / P.n_kv;
        return P.n_embed % gsz == 0 && P.n_embed / gsz <= 64 * AO_NP;
    }
}

/* phases 0 and 1 of layer l in one kernel (k_f_qkva), with AO phase 2 too */
template <int LT, class SH, int HD, int NREP, bool LONG, bool AO = false>
static void f_launch_qkva_n(const PkParams& P, const PkLayer& L, PkStep* S, int l, dim3 g, dim3 b, hipStream_t st,
                            uint8_t* atr)
{
    if constexpr (f_mixable<LT>()) {
        if (L.v) {
#define QKVA2(VT)                                                                                                    \
    do {                                                                                                             \
        if (l == 0) hipLaunchKernelGGL((k_f_qkva<LT, VT, SH, HD, NREP, true, LONG, AO>), g, b, 0, st, P, L, S, l, atr); \
        else hipLaunchKernelGGL((k_f_qkva<LT, VT, SH, HD, NREP, false, LONG, AO>), g, b, 0, st, P, L, S, l, atr);  \
    } while (0)
            if (L.v_t == LG_Q6_K_R) QKVA2(LG_Q6_K_R);
            else if (L.v_t == LG_Q6_K) QKVA2(LG_Q6_K);
            else if (L.v_t == LG_Q5_K) QKVA2(LG_Q5_K);
            else QKVA2(LT);
#undef QKVA2
            return;
        }
    }
    if (l == 0) hipLaunchKernelGGL((k_f_qkva<LT, 0, SH, HD, NREP, true, LONG, AO>), g, b, 0, st, P, L, S, l, atr);
    else hipLaunchKernelGGL((k_f_qkva<LT, 0, SH, HD, NREP, false, LONG, AO>), g, b, 0, st, P, L, S, l, atr);
}

template <int LT, class SH, int HD, int NREP>
static void f_launch_qkva(const PkParams& P, const PkLayer& L, PkStep* S, int l, dim3 g, dim3 b, hipStream_t st,
                          uint8_t* atr, bool long_ctx)
{
    if (long_ctx) f_launch_qkva_n<LT, SH, HD, NREP, true>(P, L, S, l, g, b, st, atr);
    else f_launch_qkva_n<LT, SH, HD, NREP, false>(P, L, S, l, g, b, st, atr);
}

/* phase 4 of layer l: down rows of the layer's down type */
template <int LT, class SH>
static void f_launch_down(const PkParams& P, const PkLayer& L, PkStep* S, int l, dim3 g, dim3 b, hipStream_t st,
                          uint8_t* atr)
{
    if constexpr (f_mixable<LT>()) {
        if (L.down_t != LT) {
            if (L.down_t == LG_Q6_K_R) hipLaunchKernelGGL((k_f_down<LG_Q6_K_R, SH>), g, b, 0, st, P, L, S, l, atr);
            else if (L.down_t == LG_Q6_K) hipLaunchKernelGGL((k_f_down<LG_Q6_K, SH>), g, b, 0, st, P, L, S, l, atr);
            else hipLaunchKernelGGL((k_f_down<LG_Q5_K, SH>), g, b, 0, st, P, L, S, l, atr);
            return;
        }
    }
    hipLaunchKernelGGL((k_f_down<LT, SH>), g, b, 0, st, P, L, S, l, atr);
}

template <int LT, int OT, int HD, int NREP, class SH>
static void fused_enqueue(const PkParams& P, const PkLayer* Lh, PkStep* S, int n_layers, int nwg, bool long_ctx,
                          hipStream_t st, uint8_t* atr)
{
    const dim3 g(nwg), b(PK_THREADS);
    const bool qkva = f_qkva_ok(P, nwg, long_ctx);
    if constexpr (Fmt<LT>::VALS == 64 && NREP * HD == 512 && SH::NE == 1) {
        if (f_qkvao_ok<LT, SH, HD, NREP>(P, nwg, long_ctx)) {
            /* three kernels a layer: QKV + attention + att_out by KV group,
             * up|gate on x + the partials, down */
            for (int l = 0; l < n_layers; l++) {
                if (long_ctx) f_launch_qkva_n<LT, SH, HD, NREP, true, true>(P, Lh[l], S, l, g, b, st, atr);
                else f_launch_qkva_n<LT, SH, HD, NREP, false, true>(P, Lh[l], S, l, g, b, st, atr);
                hipLaunchKernelGGL((k_f_ug<LT, SH, true>), g, b, 0, st, P, Lh[l], S, l, atr);
                f_launch_down<LT, SH>(P, Lh[l], S, l, g, b, st, atr);
            }
            f_launch_out<OT, SH>(P, S, nwg, b, st, atr);
            return;
        }
    }
    for (int l = 0; l < n_layers; l++) {
        if (qkva) {
            f_launch_qkva<LT, SH, HD, NREP>(P, Lh[l], S, l, g, b, st, atr, long_ctx);
        } else {
            f_launch_qkv<LT, SH>(P, Lh[l], S, l, g, b, st, atr);
            if (long_ctx) hipLaunchKernelGGL((k_f_attn<HD, NREP, true>), dim3(P.att_grid), b, 0, st, P, Lh[l], S, l);
            else hipLaunchKernelGGL((k_f_attn<HD, NREP, false>), g, b, 0, st, P, Lh[l], S, l);
        }
        hipLaunchKernelGGL((k_f_ao<LT, SH, HD, NREP>), g, b, 0, st, P, Lh[l], S, l, atr);
        hipLaunchKernelGGL((k_f_ug<LT, SH>), g, b, 0, st, P, Lh[l], S, l, atr);
        f_launch_down<LT, SH>(P, Lh[l], S, l, g, b, st, atr);
    }
    f_launch_out<OT, SH>(P, S, nwg, b, st, atr);
}

typedef void (*fused_phase_t)(const PkParams&, const PkLayer*, PkStep*, int, int, int, bool, hipStream_t);

/* one kernel of the step: phase 0..4 of layer l, 5 = output head */
template <int LT, int OT, int HD, int NREP, class SH>
static void fused_phase(const PkParams& P, const PkLayer* Lh, PkStep* S, int phase, int l, int nwg, bool long_ctx,
                        hipStream_t st)
{
    const dim3 g(nwg), b(PK_THREADS);
    bool ao = false;
    if constexpr (Fmt<LT>::VALS == 64 && NREP * HD == 512 && SH::NE == 1) ao = f_qkvao_ok<LT, SH, HD, NREP>(P, nwg, long_ctx);
    switch (phase) {
    case 0:   /* with the fused QKV + attention (+ att_out) kernel in use, that kernel */
        if constexpr (Fmt<LT>::VALS == 64 && NREP * HD == 512 && SH::NE == 1) {
            if (ao) {
                if (long_ctx) f_launch_qkva_n<LT, SH, HD, NREP, true, true>(P, Lh[l], S, l, g, b, st, nullptr);
                else f_launch_qkva_n<LT, SH, HD, NREP, false, true>(P, Lh[l], S, l, g, b, st, nullptr);
                break;
            }
        }
        if (f_qkva_ok(P, nwg, long_ctx)) f_launch_qkva<LT, SH, HD, NREP>(P, Lh[l], S, l, g, b, st, nullptr, long_ctx);
        else f_launch_qkv<LT, SH>(P, Lh[l], S, l, g, b, st, nullptr);
        break;
    case 1:
        if (long_ctx) hipLaunchKernelGGL((k_f_attn<HD, NREP, true>), dim3(P.att_grid), b, 0, st, P, Lh[l], S, l);
        else hipLaunchKernelGGL((k_f_attn<HD, NREP, false>), g, b, 0, st, P, Lh[l], S, l);
        break;
    case 2: hipLaunchKernelGGL((k_f_ao<LT, SH, HD, NREP>), g, b, 0, st, P, Lh[l], S, l, nullptr); break;
    case 3:   /* the up|gate kernel the step runs */
        if constexpr (Fmt<LT>::VALS == 64 && NREP * HD == 512 && SH::NE == 1) {
            if (ao) { hipLaunchKernelGGL((k_f_ug<LT, SH, true>), g, b, 0, st, P, Lh[l], S, l, nullptr); break; }
        }
        hipLaunchKernelGGL((k_f_ug<LT, SH>), g, b, 0, st, P, Lh[l], S, l, nullptr);
        break;
    case 4: f_launch_down<LT, SH>(P, Lh[l], S, l, g, b, st, nullptr); break;
    default: f_launch_out<OT, SH>(P, S, nwg, b, st, nullptr); break;
    }
}

/* slots per lane of a row of n values of type t, and 256-value chunks per
 * wave of an n-wide activation build */
static constexpr int f_vps(int t) { return (t == LG_Q8_0 || t == LG_Q1_0 || t == LG_F16 || t == LG_F32) ? 32 : 64; }
/* the kernels' form of a file type: F16 / F32 rows dot an fp32 activation
 * held in LDS (Fmt<LG_F16_L>, Fmt<LG_F32_L>) */
static constexpr int f_kt(int t) { return t == LG_F16 ? LG_F16_L : t == LG_F32 ? LG_F32_L : t; }
static constexpr int f_ns(int t, int n) { return (n / f_vps(t) + 63) / 64; }
static constexpr int f_cpw(int n) { return (n + 256 * PK_WAVES - 1) / (256 * PK_WAVES); }

struct FusedVariant {
    int lt, ot, hd, nrep;
    int ne, no, ce, nf, cf;       /* the FShape */
    fused_enqueue_t fn;
    fused_phase_t phase;
    fused_enqueue_t fn_r;         /* the same on regrouped layer matrices (PkParams.layers_rep) */
    fused_phase_t phase_r;
};

/* one variant per (layer type, output type, head_dim, query heads per KV
 * head) and width class: n_embed 4096 / n_ff 12288 (the Qwen3-8B shape),
 * n_embed 4096 / n_ff 14336 (Llama-3-8B, Mistral-7B), n_embed 2560 / n_ff
 * 9728 (Qwen3-4B), n_embed 5120 / n_ff 17408 (Qwen3-14B: 40 query heads on
 * 8 KV heads), n_embed 2048 / n_ff 5632 (TinyLlama-1.1B, head_dim 64), and
 * any width up to 2048 / 2048 (tiny models); F16 and F32 layers (and head)
 * at the Qwen3-8B shape */
#define FVS(LT, OT, HD, NR, E, F)                                                                              \
    {LT, OT, HD, NR, f_ns(LT, E), f_ns(OT, E), f_cpw(E), f_ns(LT, F), f_cpw(F),                                \
     fused_enqueue<f_kt(LT), f_kt(OT), HD, NR, FShape<f_ns(LT, E), f_ns(OT, E), f_cpw(E), f_ns(LT, F), f_cpw(F)>>,  \
     fused_phase<f_kt(LT), f_kt(OT), HD, NR, FShape<f_ns(LT, E), f_ns(OT, E), f_cpw(E), f_ns(LT, F), f_cpw(F)>>,    \
     fused_enqueue<f_rep(f_kt(LT)), f_kt(OT), HD, NR,                                                          \
                   FShape<f_ns(LT, E), f_ns(OT, E), f_cpw(E), f_ns(LT, F), f_cpw(F)>>,                         \
     fused_phase<f_rep(f_kt(LT)), f_kt(OT), HD, NR, FShape<f_ns(LT, E), f_ns(OT, E), f_cpw(E), f_ns(LT, F), f_cpw(F)>>}
#define FV(LT, OT, HD, NR) FVS(LT, OT, HD, NR, 4096, 12288)
/* the table in four parts, one per translation unit (lg_fused.hip and
 * lg_fused_p1..p3.hip, which include this file with LG_FUSED_PART set), so
 * that the variants compile in parallel */
#ifndef LG_FUSED_PART
#define LG_FUSED_PART 0
#endif
#if LG_FUSED_PART == 0
const FusedVariant* lg_fused_part_0(int* n)
{
    static const FusedVariant v[] = {
        FV(LG_Q4_K, LG_Q6_K, 128, 4), FV(LG_Q4_K, LG_Q4_K, 128, 4), FV(LG_Q4_K, LG_Q8_0, 128, 4),
        FV(LG_Q5_K, LG_Q6_K, 128, 4), FV(LG_Q6_K, LG_Q6_K, 128, 4), FV(LG_Q8_0, LG_Q8_0, 128, 4),
        FV(LG_F16, LG_Q6_K, 128, 4),
    };
    *n = (int)(sizeof(v) / sizeof(v[0]));
    return v;
}
#elif LG_FUSED_PART == 1
const FusedVariant* lg_fused_part_1(int* n)
{
    static const FusedVariant v[] = {
        FV(LG_Q1_G, LG_Q8_0, 128, 4), FV(LG_Q1_G, LG_Q6_K, 128, 4), FV(LG_Q3_K, LG_Q6_K, 128, 4),
        FV(LG_Q2_K, LG_Q6_K, 128, 4), FV(LG_Q8_0, LG_Q6_K, 128, 4), FV(LG_Q1_0, LG_Q8_0, 128, 4),
        FV(LG_Q8_0, LG_Q8_0, 128, 1),
    };
    *n = (int)(sizeof(v) / sizeof(v[0]));
    return v;
}
#elif LG_FUSED_PART == 2
const FusedVariant* lg_fused_part_2(int* n)
{
    static const FusedVariant v[] = {
        FV(LG_Q4_K, LG_Q6_K, 128, 8), FV(LG_Q4_K, LG_Q6_K, 128, 1), FV(LG_Q5_K, LG_Q4_K, 128, 1),
        FV(LG_Q5_K, LG_Q6_K, 128, 8),
        FVS(LG_Q4_K, LG_Q6_K, 128, 4, 4096, 14336), FVS(LG_Q8_0, LG_Q8_0, 128, 4, 4096, 14336),
        FV(LG_F16, LG_F16, 128, 4),
    };
    *n = (int)(sizeof(v) / sizeof(v[0]));
    return v;
}
#else
const FusedVariant* lg_fused_part_3(int* n)
{
    static const FusedVariant v[] = {
        FVS(LG_Q4_K, LG_Q6_K, 128, 4, 2560, 9728), FVS(LG_Q4_K, LG_Q6_K, 128, 5, 5120, 17408),
        FVS(LG_Q4_K, LG_Q6_K, 64, 8, 2048, 5632), FVS(LG_Q8_0, LG_Q8_0, 64, 8, 2048, 5632),
        FVS(LG_Q8_0, LG_Q8_0, 48, 1, 2048, 2048), FVS(LG_Q8_0, LG_Q8_0, 64, 1, 2048, 2048),
        FVS(LG_Q4_K, LG_Q6_K, 64, 1, 2048, 2048), FV(LG_F32, LG_F32, 128, 4),
    };
    *n = (int)(sizeof(v) / sizeof(v[0]));
    return v;
}
#endif
#undef FV
#undef FVS

#if LG_FUSED_PART == 0
const FusedVariant* lg_fused_part_1(int* n);
const FusedVariant* lg_fused_part_2(int* n);
const FusedVariant* lg_fused_part_3(int* n);
struct FusedPart {
    const FusedVariant* v;
    int n;
};

const void* lg_fused_variant(int lt, int ot, int hd, int nrep, int ne, int nff)
{
    FusedPart f_parts[4];
    f_parts[0].v = lg_fused_part_0(&f_parts[0].n);
    f_parts[1].v = lg_fused_part_1(&f_parts[1].n);
    f_parts[2].v = lg_fused_part_2(&f_parts[2].n);
    f_parts[3].v = lg_fused_part_3(&f_parts[3].n);
    /* a variant serves the model when its slots and chunks hold the model's
     * widths (masked past them) and it wastes no more than its class does */
    for (const FusedPart& fp : f_parts)
        for (int k = 0; k < fp.n; k++) {
            const FusedVariant& v = fp.v[k];
            if (v.lt != lt || v.ot != ot || v.hd != hd || v.nrep != nrep) continue;
            if (f_ns(lt, ne) == v.ne && f_ns(ot, ne) == v.no && f_cpw(ne) == v.ce && f_ns(lt, nff) == v.nf &&
                f_cpw(nff) == v.cf)
                return (const void*)&v;
        }
    for (const FusedPart& fp : f_parts)
        for (int k = 0; k < fp.n; k++) {
            const FusedVariant& v = fp.v[k];
            if (v.lt != lt || v.ot != ot || v.hd != hd || v.nrep != nrep) continue;
            if (f_ns(lt, ne) <= v.ne && f_ns(ot, ne) <= v.no && f_cpw(ne) <= v.ce && f_ns(lt, nff) <= v.nf &&
                f_cpw(nff) <= v.cf && v.ce <= 1 && v.cf <= 1)
                return (const void*)&v;
        }
    return nullptr;
}

int lg_fused_enqueue(const void* variant, const PkParams& P, const PkLayer* layers, PkStep* S_dev, int n_layers, int nwg,
                     bool long_ctx, hipStream_t s, uint8_t* act_trace)
{
    const FusedVariant* v = (const FusedVariant*)variant;
    (P.layers_rep ? v->fn_r : v->fn)(P, layers, S_dev, n_layers, nwg, long_ctx, s, act_trace);
    return lg_check_launch("fused decode step");
}

int lg_fused_phase(const void* variant, const PkParams& P, const PkLayer* layers, PkStep* S_dev, int phase, int layer,
                   int nwg, bool long_ctx, hipStream_t s)
{
    const FusedVariant* v = (const FusedVariant*)variant;
    (P.layers_rep ? v->phase_r : v->phase)(P, layers, S_dev, phase, layer, nwg, long_ctx, s);
    return lg_check_launch("fused decode phase");
}
#endif   /* LG_FUSED_PART == 0 */
