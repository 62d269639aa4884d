/* lg_persist.hip -- the whole per-token step of inference()
 * (fast/ligguf_fast_qk.cpp:24-144) as ONE persistent kernel for gfx950.
 *
 * Why.  A batch-1 token of an 8B model is ~400 small dependent operations;
 * as separate kernels each pays launch, ramp and end-of-kernel cache
 * write-back (a few microseconds apiece), which dominates the 0.56 ms that
 * HBM needs for the weights.  Here one cooperative launch of one workgroup
 * per CU (8 waves) walks the layer loop; the phases are separated by
 * flag syncs, and every wave issues the loads of its next weight rows
 * BEFORE it waits for the activation they multiply, so the weight stream
 * keeps running through the syncs.
 *
 * Phases per layer l (dependencies are on all workgroups' progress):
 *   A  rmsnorm(x)->Q8 in LDS (every WG), QKV matvec rows       -> qkv
 *   B  attention units (kv head g, sequence chunk c): QK-norm, RoPE and the
 *      fp16 KV write of row pos, scores/softmax/PV partials; the last unit
 *      of a head (atomic counter) merges its partials          -> att
 *   C  Q8(att) in LDS, att_out rows, x[r] += ...              -> x
 *   D  rmsnorm(x)->Q8, up|gate row pairs, SwiGLU              -> hb
 *   E  Q8(hb) in LDS, down rows, x[r] += ...                  -> x
 * then F: rmsnorm(x)->Q8, output rows -> logits, per-WG argmax, and the last
 * WG reduces the argmax (sampler_greedy, fast/ligguf_fast_qk.cpp:146-160).
 *
 * Cross-workgroup data.  Everything one WG writes for another (qkv, att, x,
 * hb, attention partials, argmax partials) is stored and loaded with
 * agent-scope relaxed atomics (global_store/load ... sc1: write-through /
 * coherent at the device level, no L2 write-back or invalidate), and a WG
 * publishes a phase only after `s_waitcnt vmcnt(0)` in every wave (all its
 * stores acknowledged) and a workgroup barrier; then one lane stores the
 * WG's 64-bit progress word.  Waiting = one wave polling the minimum of all
 * progress words.  Every wait is bounded: on expiry the kernel records an
 * error flag, stops waiting and runs to the end, so it always terminates;
 * the host turns the flag into LG_ERR_STATE.
 *
 * Numerics are those of the multi-kernel path (same slot order, same lane
 * reductions, same quantizers), so both paths give the same bits wherever
 * their work split agrees (the matvecs, norms, SwiGLU); attention splits
 * the sequence differently, which changes fp32 rounding only.
 */
#include <hip/hip_runtime.h>

/* the thread index through an empty asm, once per use (see lg_phase.h) */
static __device__ __forceinline__ int pk_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
#define LG_TID pk_tid()
#include "lg_phase.h"

/* ------------------------------------------------------------------ */
/* the kernel                                                           */
/* ------------------------------------------------------------------ */
/* layer l from the per-kind arenas: pointers computed from kernel
 * arguments, so the weight loads stay global (not flat) loads */
__device__ __forceinline__ PkLayer pk_layer(const PkParams& P, int l)
{
    PkLayer L;
    L.qkv = P.w_qkv + (size_t)l * P.s_qkv;
    L.ao = P.w_ao + (size_t)l * P.s_ao;
    L.ug = P.w_ug + (size_t)l * P.s_ug;
    L.down = P.w_down + (size_t)l * P.s_down;
    L.qkv_rsz = (uint32_t)(P.s_qkv / (P.n_embed + 2 * P.kv_dim));
    L.ao_rsz = (uint32_t)(P.s_ao / P.n_embed);
    L.ug_rsz = (uint32_t)(P.s_ug / (2 * P.n_ff));
    L.down_rsz = (uint32_t)(P.s_down / P.n_embed);
    L.qkv_t = L.ao_t = L.ug_t = L.down_t = 0;   /* the kernel's template type */
    L.att_norm = P.n_att + (size_t)l * P.n_embed;
    L.ffn_norm = P.n_ffn + (size_t)l * P.n_embed;
    L.q_norm = P.n_q ? P.n_q + (size_t)l * P.head_dim : nullptr;
    L.k_norm = P.n_k ? P.n_k + (size_t)l * P.head_dim : nullptr;
    return L;
}

/* One instantiation per (layer type, output type, head_dim, query heads per
 * KV head), for n_embed 4096 and n_ff 12288 (the engine checks the widths): every phase body is inlined, so no call saves registers, and the
 * phases use the matvec batch sizes of the fused kernels (no spills: the
 * opaque thread index above keeps per-phase address arithmetic inside the
 * layer loop).  Activation buffers (each written once per launch): xs[l] =
 * residual stream entering layer l (xs[0] the embedding row, xs[L] the output
 * of the last layer), xm[l] = after attention, qkv[l], hb[l]; the attention
 * partials (att_po/att_pml) are per layer too. */
template <int LT, int OT, int HD, int NREP>
__global__ __launch_bounds__(PK_THREADS) void k_decode_persistent(const PkParams P, PkStep S)
{
    const int ne = P.n_embed, kvd = P.kv_dim, nff = P.n_ff;
    const int qs = ne + 2 * kvd;
    const uint64_t B = S.base;
    constexpr int NE = NsE<LT>::value, NF = 3 * NE;
#define TR(p) (S.trace ? S.trace + ((size_t)(p) * gridDim.x + blockIdx.x) * 4 : nullptr)
#define ATR(k) (S.act_trace ? S.act_trace + (size_t)(k) * P.act_stride : nullptr)
    /* a step queued behind another without a host round trip takes the
     * greedy token the step before it left in tok_out */
    const int tok = S.tok >= 0 ? S.tok : __builtin_amdgcn_readfirstlane(cld(P.tok_out));
    for (int l = 0; l < P.n_layers; l++) {
        const PkLayer L = pk_layer(P, l);
        const uint64_t p0 = B + 5ull * l;
        float* xin = P.xs + (size_t)l * ne;
        float* xmid = P.xm + (size_t)l * ne;
        float* xout = P.xs + (size_t)(l + 1) * ne;
        float* qkv = P.qkv + (size_t)l * qs;
        float* hb = P.hb + (size_t)l * nff;
        if (l == 0)
            phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, BLD_EMB, 2, LG_QKV_R>(
                P, tok, L.qkv, L.qkv_rsz, qs, 0, L.att_norm, xin, nullptr, qkv, xin, 0, p0 + 1, TR(5 * l), ATR(4 * l), ne);
        else
            phase_mv<LT, NE, LG_QKV_B, 1, EPI_STORE, BLD_RMS, 2, LG_QKV_R>(
                P, tok, L.qkv, L.qkv_rsz, qs, 0, L.att_norm, xin, nullptr, qkv, xin, p0, p0 + 1, TR(5 * l), ATR(4 * l), ne);
        phase_attn_any<HD, NREP>(P, L, l, S.pos, qkv, p0 + 1, p0 + 2, TR(5 * l + 1));
        phase_mv<LT, NE, LG_AO_B, 1, EPI_RESID, BLD_MERGE, 2, LG_AO_R>(
            P, 0, L.ao, L.ao_rsz, ne, 0, nullptr, nullptr, xin, xmid, nullptr, p0 + 2, p0 + 3, TR(5 * l + 2),
            ATR(4 * l + 1), ne, att_partials<HD, NREP>(P, l, S.pos));
        phase_mv<LT, NE, LG_UG_B, 2, EPI_SWIGLU, BLD_RMS, 2, LG_UG_R>(
            P, 0, L.ug, L.ug_rsz, nff, nff, L.ffn_norm, xmid, nullptr, hb, nullptr, p0 + 3, p0 + 4, TR(5 * l + 3),
            ATR(4 * l + 2), ne);
        phase_mv<LT, NF, LG_DN_B, 1, EPI_RESID, BLD_PLAIN, 6, LG_DN_R>(
            P, 0, L.down, L.down_rsz, ne, 0, nullptr, hb, xmid, xout, nullptr, p0 + 4, p0 + 5, TR(5 * l + 4),
            ATR(4 * l + 3), nff);
    }
    const uint64_t pf = B + 5ull * P.n_layers;
    constexpr int NO = NsE<OT>::value;
    phase_mv<OT, NO, LG_OUT_B, 1, EPI_LOGITS, BLD_RMS, 2, LG_OUT_R>(
        P, 0, P.out_w, P.out_rsz, P.vocab, 0, P.out_norm, P.xs + (size_t)P.n_layers * ne, nullptr, P.logits, nullptr,
        pf, pf + 1, TR(5 * P.n_layers), ATR(4 * P.n_layers), ne);
    /* s_int[0]: this workgroup reduced the argmax and wrote tok_out */
    if (s_int[0] && LG_TID == 0) cst(&P.tok_hist[S.pos], cld(P.tok_out));
#undef TR
#undef ATR
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */
typedef void (*pk_kernel_t)(const PkParams, PkStep);

struct PkVariant {
    int lt, ot, hd, nrep;
    pk_kernel_t fn;
};

#define PKV(LT, OT, HD, NR) {LT, OT, HD, NR, k_decode_persistent<LT, OT, HD, NR>}
static const PkVariant k_variants[] = {
    PKV(LG_Q4_K, LG_Q6_K, 128, 4), PKV(LG_Q4_K, LG_Q4_K, 128, 4), PKV(LG_Q4_K, LG_Q8_0, 128, 4),
    PKV(LG_Q5_K, LG_Q6_K, 128, 4), PKV(LG_Q6_K, LG_Q6_K, 128, 4), PKV(LG_Q8_0, LG_Q8_0, 128, 4),
    PKV(LG_Q1_G, LG_Q8_0, 128, 4), PKV(LG_Q1_G, LG_Q6_K, 128, 4),
    PKV(LG_Q4_K, LG_Q6_K, 128, 8), PKV(LG_Q4_K, LG_Q6_K, 128, 1), PKV(LG_Q5_K, LG_Q4_K, 128, 1),
    PKV(LG_Q8_0, LG_Q8_0, 128, 1),
};
#undef PKV

const void* lg_persist_kernel(int lt, int ot, int hd, int nrep)
{
    for (const PkVariant& v : k_variants)
        if (v.lt == lt && v.ot == ot && v.hd == hd && v.nrep == nrep) return (const void*)v.fn;
    return nullptr;
}

int lg_persist_grid(const void* kernel, int* nwg)
{
    int dev = 0, ncu = 0, per = 0;
    LG_HIP_CHECK(hipGetDevice(&dev));
    LG_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    LG_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, PK_THREADS, 0));
    if (per < 1) {
        lg_set_error("persistent decode kernel does not fit on a CU");
        return LG_ERR_HIP;
    }
    *nwg = ncu;
    return LG_OK;
}

int lg_persist_launch(const void* kernel, const PkParams& P, const PkStep* S, int nwg, hipStream_t s)
{
    PkParams p = P;
    PkStep st = *S;
    void* args[] = {&p, &st};
    LG_HIP_CHECK(hipLaunchCooperativeKernel(kernel, dim3(nwg), dim3(PK_THREADS), args, 0, s));
    return LG_OK;
}
