/* lg_persist.h -- parameters of the persistent per-token decode kernel
 * (lg_persist.hip), filled by the engine (lg_engine.hip). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PK_THREADS 512      /* 8 waves per workgroup, one workgroup per CU */
#define PK_MAX_EMBED 8192   /* n_embed limit (fp32 staging of x in LDS) */
#define PK_MAX_FF 20480     /* n_ff limit (quantized activation in LDS) */
#define PK_MAX_FF_F 12288   /* n_ff limit of F16 / F32 layers (fp32 activation in LDS) */
#define PK_MAX_NREP 8       /* query heads per KV head */
#define PK_ATT_MERGE 8      /* attention partials per head merged by the att_out build */
#define LG_MAX_GROUP_WORDS 1024 /* workgroups of the fused QKV + attention kernel, at most (one barrier word each) */
#define PK_ATT_MAX_NCH 160  /* attention chunks per head at most */
#define LG_OUT_MAX_WGS 4     /* output-head workgroups per CU at most (argmax partials) */
/* long-context attention workgroups per CU: with 2 the fused step's kernel
 * runs two side by side at 128 VGPRs (half the chunk length, q from LDS)
 * and the persistent kernel takes the same units in turn, so both compute
 * the same chunks; measured slower than one (Q1_G 8192-context decode 442
 * against 478 tok/s), so one */
#ifndef LG_ATT_WGS
#define LG_ATT_WGS 1
#endif

/* one layer as the kernels read it: fused Q|K|V and up|gate matrices; in
 * the fused step's mixed layers (v != NULL) qkv is Q|K and V a matrix of
 * its own type v_t, and down_t may differ from the layer type */
struct PkLayer {
    const uint8_t* qkv;
    const uint8_t* ao;
    const uint8_t* ug;
    const uint8_t* down;
    uint32_t qkv_rsz, ao_rsz, ug_rsz, down_rsz;
    int qkv_t, ao_t, ug_t, down_t;
    const float* att_norm;
    const float* ffn_norm;
    const float* q_norm;     /* NULL for llama */
    const float* k_norm;
    const uint8_t* v;        /* NULL: V is part of qkv */
    uint32_t v_rsz;
    int v_t;
};

struct PkParams {
    const PkLayer* layers;
    /* the same layers as per-kind arenas, layer l at base + l * stride (the
     * persistent kernel derives its layer from these kernel arguments);
     * w_qkv NULL when the model's layers differ in shape or type */
    const uint8_t *w_qkv, *w_ao, *w_ug, *w_down;
    uint64_t s_qkv, s_ao, s_ug, s_down;
    const float *n_att, *n_ffn, *n_q, *n_k;   /* strides n_embed, n_embed, head_dim, head_dim */
    int n_layers, n_embed, n_heads, n_kv, head_dim, kv_dim, n_ff, vocab, n_ctx, rope_dim;
    float eps;
    const uint8_t* embd;
    uint32_t embd_rsz;
    int embd_t;
    const uint8_t* out_w;
    const uint8_t* out_wr;    /* the output head regrouped for aligned loads (repack_rows), or NULL */
    int layers_rep;           /* the fused step's PkLayer matrices are regrouped copies (Q8_0, Q6_K, Q1_G layers) */
    uint32_t out_rsz;
    int out_t;
    const float* out_norm;
    const float* rope_freq;
    uint16_t* kc;
    uint16_t* vc;
    float* xs;               /* [n_layers+1][n_embed] residual stream entering each layer */
    float* xm;               /* [n_layers][n_embed] after the attention residual */
    float* qkv;              /* [n_layers][n_embed + 2*kv_dim] */
    float* hb;               /* [n_layers][n_ff] */
    float* logits;
    float* att_po;           /* [n_layers][att_slots][n_embed] unnormalised attention partials */
    float* att_pml;          /* [n_layers][att_slots][n_heads][2] their (max, sum), log2 units */
    int att_slots;           /* per layer: one per chunk, then PK_ATT_MERGE for the groups merged in-kernel */
    int att_grid;            /* long-context split: units sized for this many workgroups (LG_ATT_WGS per CU) */
    uint32_t* attn_cnt;      /* [unit head sets (n_kv * NREP / NQ <= 32)][PK_ATT_MERGE groups], zero between launches */
    uint64_t* grp_cnt;       /* [LG_MAX_GROUP_WORDS] KV-group barrier words of the fused QKV + attention kernel (launch counts) */
    int qkva;                /* fused path: QKV and short-context attention in one kernel (LG_NO_QKVA=1: two) */
    int qkvao;               /* fused path: att_out in that kernel too, split by KV group (LG_NO_QKVAO=1: its own kernel) */
    float* ao_part;          /* [8][n_embed] att_out partials of the KV groups, summed by the next up|gate build */
    uint64_t* progress;      /* one word per workgroup */
    float* amax_v;           /* per-workgroup argmax partials */
    int* amax_i;
    uint32_t* amax_cnt;      /* zero between launches */
    int* tok_out;            /* greedy token of this step */
    int* tok_hist;           /* [n_ctx]: the greedy token of the step at each position */
    uint32_t* err;           /* nonzero: a sync wait expired (or an unsupported phase) */
    const int* feed;         /* [n_ctx] prompt tokens for positions < PkStep.feed_end (fused path) */
    int spin_cap;
    uint64_t act_stride;     /* bytes per slot of an activation trace */
};

/* what changes from token to token (PkParams, fixed per model, and PkStep
 * are kernel arguments; the fused kernels read PkStep from device memory) */
struct PkStep {
    int tok, pos;            /* persistent kernel: tok < 0 takes the previous step's greedy token (tok_out) */
    int feed_end;            /* fused path: positions below this take their token from PkParams.feed */
    int pad_;
    uint64_t base;           /* progress value at launch; the launch adds 5*n_layers + 1 */
    uint64_t* trace;         /* NULL, or [5*n_layers+1][gridDim][4] timestamps (100 MHz clock):
                                phase entry, wait done, activation built, phase published */
    uint8_t* act_trace;      /* persistent kernel: NULL, or [4*n_layers+1][PkParams.act_stride] bytes:
                                every quantized activation of the step as workgroup 0 built it (per
                                layer: attention input, attention output, FFN input, SwiGLU output;
                                then the output head's input), in its GGUF block layout (the fused
                                kernels take the same pointer as a kernel argument) */
};

/* the head width the attention lanes are laid out for: a position takes
 * pk_hdp / 8 lanes of 8 values (a power of two; head_dim 48 runs as 64 with
 * its last 16 values zero) */
__host__ __device__ constexpr int pk_hdp(int head_dim)
{
    return head_dim <= 64 ? 64 : 128;
}

/* attention work split.  A workgroup step covers ppb = PK_THREADS * 8 /
 * pk_hdp(head_dim) positions (one 16-byte slice of a cache row per lane) and a unit
 * (kv head, chunk) holds pk_att_steps(nrep) steps of K and V in registers at
 * a time -- one register batch.  Contexts up to PK_ATT_MERGE batches are cut
 * into at most PK_ATT_MERGE chunks per head, whose partials the att_out build
 * merges; longer ones into max_nch chunks (the grid's workgroups per head
 * group, clamped to [PK_ATT_MERGE, PK_ATT_MAX_NCH]) of one or more batches,
 * merged in at most PK_ATT_MERGE groups of pk_att_group chunks (by the last
 * unit of each group), the att_out build merging the groups. */
__host__ __device__ constexpr int pk_att_steps(int nrep)
{
    return nrep > 4 ? 4 : 8;
}

/* query heads per attention unit.  One, while every unit of the phase gets a
 * workgroup of its own (n_kv x NREP x chunks <= grid): a unit carries 1/NREP
 * of the group's arithmetic (its work is lane arithmetic, not memory), so
 * NREP times as many workgroups share the phase, and the NREP units that read
 * the same K/V rows run at the same time on one XCD, whose L2 serves the
 * repeats.  Past that (long contexts) a unit takes all NREP query heads, so
 * every K/V row is read from HBM once. */
__host__ __device__ inline bool pk_att_one_head(int n_kv, int nrep, int nch, int nwg)
{
    return n_kv * nrep * nch <= nwg;
}

__host__ __device__ inline void pk_attn_split(int ctx_len, int head_dim, int nrep, int max_nch, int* chunk_out,
                                              int* nch_out)
{
    const int ppb = PK_THREADS * 8 / pk_hdp(head_dim);
    int chunk = (ctx_len + PK_ATT_MERGE - 1) / PK_ATT_MERGE;
    chunk = (chunk + ppb - 1) / ppb * ppb;
    if (chunk > pk_att_steps(nrep) * ppb) {
        const int n = max_nch < PK_ATT_MERGE ? PK_ATT_MERGE : (max_nch > PK_ATT_MAX_NCH ? PK_ATT_MAX_NCH : max_nch);
        chunk = (ctx_len + n - 1) / n;
        chunk = (chunk + ppb - 1) / ppb * ppb;
    }
    *chunk_out = chunk;
    *nch_out = (ctx_len + chunk - 1) / chunk;
}

/* long contexts: chunks per merge group and the group count (<= PK_ATT_MERGE) */
__host__ __device__ constexpr int pk_att_group(int nch)
{
    return (nch + PK_ATT_MERGE - 1) / PK_ATT_MERGE;
}
__host__ __device__ constexpr int pk_att_ngroups(int nch)
{
    return (nch + pk_att_group(nch) - 1) / pk_att_group(nch);
}

/* the kernel instantiated for (layer type, output type, head_dim, query heads
 * per KV head), or NULL: the model then runs on the multi-kernel path */
const void* lg_persist_kernel(int layer_type, int out_type, int head_dim, int nrep);
int lg_persist_grid(const void* kernel, int* nwg);
int lg_persist_launch(const void* kernel, const PkParams& P, const PkStep* S, int nwg, hipStream_t s);

/* short contexts: chunks of a fixed pk_att_fch positions (one register
 * batch at most), one query head per unit, unit u = (kv head u % n_kv,
 * query head (u / n_kv) % nrep of its group, chunk u / n_heads).  No part of
 * a unit's rows depends on the step's position, so its loads are issued
 * before the position arrives (the fused kernels read it from memory);
 * units past the context skip their work. */
__host__ __device__ constexpr int pk_att_fch(int head_dim, int nrep)
{
    return pk_att_steps(nrep) * (PK_THREADS * 8 / pk_hdp(head_dim)) < 128
               ? pk_att_steps(nrep) * (PK_THREADS * 8 / pk_hdp(head_dim))
               : 128;
}

/* attention at position pos takes the long-context units (whole query-head
 * groups, register batches, pk_attn_split) unless the context fits
 * PK_ATT_MERGE fixed chunks and every short unit has a workgroup of its own */
__host__ __device__ inline bool pk_att_long(int pos, int head_dim, int nrep, int n_kv, int nwg)
{
    return !(pos + 1 <= PK_ATT_MERGE * pk_att_fch(head_dim, nrep) && pk_att_one_head(n_kv, nrep, PK_ATT_MERGE, nwg));
}

/* the fused per-phase kernels of one step (lg_fused.hip): 5*n_layers + 1
 * launches on stream s reading {tok, pos} from S_dev; the last one writes the
 * greedy token to P->tok_out and advances S_dev to {token, pos + 1}.  NULL
 * when the variant is not instantiated.  long_ctx = pk_att_long(pos, ...) of
 * the step's position selects the attention kernel. */
const void* lg_fused_variant(int layer_type, int out_type, int head_dim, int nrep, int n_embed, int n_ff);
/* whether the fused step takes a V or down matrix of type t among layers of
 * layer_type (Q4_K_M / Q4_K_S / Q5_K_M-style mixes: Q5_K or Q6_K among Q4_K
 * or Q5_K layers) */
bool lg_fused_side_type(int layer_type, int t);
int lg_fused_enqueue(const void* variant, const PkParams& P, const PkLayer* layers, PkStep* S_dev, int n_layers, int nwg,
                     bool long_ctx, hipStream_t s, uint8_t* act_trace = nullptr);
/* one kernel of the fused step: phase 0 rmsnorm+QKV, 1 attention, 2 att_out,
 * 3 up|gate, 4 down (of `layer`), 5 output head */
int lg_fused_phase(const void* variant, const PkParams& P, const PkLayer* layers, PkStep* S_dev, int phase, int layer,
                   int nwg, bool long_ctx, hipStream_t s);
