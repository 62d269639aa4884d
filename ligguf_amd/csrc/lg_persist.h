/* lg_persist.h -- parameters of the persistent per-token decode kernel
 * (lg_persist.hip), filled by the engine (lg_engine.hip). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PK_THREADS 512      /* 8 waves per workgroup, one workgroup per CU */
#define PK_MAX_EMBED 8192   /* n_embed limit (fp32 staging of x in LDS) */
#define PK_MAX_FF 16384     /* n_ff limit (quantized activation in LDS) */
#define PK_MAX_NREP 8       /* query heads per KV head */
#define PK_MAX_CHUNK 512    /* attention positions per unit */
#define PK_MAX_UNITS_PER_HEAD 64

/* one layer as the kernel reads it: fused Q|K|V and up|gate matrices */
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
};

struct PkParams {
    const PkLayer* layers;
    int n_layers, n_embed, n_heads, n_kv, head_dim, kv_dim, n_ff, vocab, n_ctx, rope_dim;
    float eps;
    const uint8_t* embd;
    uint32_t embd_rsz;
    int embd_t;
    const uint8_t* out_w;
    uint32_t out_rsz;
    int out_t;
    const float* out_norm;
    const float* rope_freq;
    uint16_t* kc;
    uint16_t* vc;
    float* xs;               /* [n_layers+1][n_embed] residual stream entering each layer */
    float* xm;               /* [n_layers][n_embed] after the attention residual */
    float* qkv;              /* [n_layers][n_embed + 2*kv_dim] */
    float* att;              /* [n_layers][n_embed] */
    float* hb;               /* [n_layers][n_ff] */
    float* logits;
    float* attn_ws;          /* n_kv * PK_MAX_UNITS_PER_HEAD partials of NREP*(head_dim+2) floats */
    uint32_t* attn_cnt;      /* n_kv counters, zero between launches */
    uint64_t* progress;      /* one word per workgroup */
    float* amax_v;           /* per-workgroup argmax partials */
    int* amax_i;
    uint32_t* amax_cnt;      /* zero between launches */
    int* tok_out;            /* greedy token of this step */
    uint32_t* err;           /* nonzero: a sync wait expired (or an unsupported phase) */
    const int* feed;         /* [n_ctx] prompt tokens for positions < PkStep.feed_end (fused path) */
    int spin_cap;
};

/* what changes from token to token (a kernel argument; PkParams lives in
 * device memory, uploaded once per model) */
struct PkStep {
    int tok, pos, nch, chunk;
    int feed_end;            /* fused path: positions below this take their token from PkParams.feed */
    int pad_;
    uint64_t base;           /* progress value at launch; the launch adds 5*n_layers + 1 */
    uint64_t* trace;         /* NULL, or [5*n_layers+1][gridDim][4] timestamps (100 MHz clock):
                                phase entry, wait done, activation built, phase published */
};

/* attention work split for a context of ctx_len positions: units of
 * (kv head, chunk) of about one per workgroup, 64..PK_MAX_CHUNK positions */
__host__ __device__ inline void pk_attn_split(int ctx_len, int n_kv, int nwg, int* chunk_out, int* nch_out)
{
    int chunk = (int)(((long long)ctx_len * n_kv + nwg - 1) / nwg);
    chunk = (chunk + 31) / 32 * 32;
    if (chunk < 64) chunk = 64;
    if (chunk > PK_MAX_CHUNK) chunk = PK_MAX_CHUNK;
    *chunk_out = chunk;
    *nch_out = (ctx_len + chunk - 1) / chunk;
}

/* the kernel instantiated for (layer type, output type, head_dim, query heads
 * per KV head), or NULL: the model then runs on the multi-kernel path */
const void* lg_persist_kernel(int layer_type, int out_type, int head_dim, int nrep);
int lg_persist_grid(const void* kernel, int* nwg);
int lg_persist_launch(const void* kernel, const PkParams* P_dev, const PkStep* S, int nwg, hipStream_t s);

/* the fused per-phase kernels of one step (lg_fused.hip): 5*n_layers + 1
 * launches on stream s reading {tok, pos} from S_dev; the last one writes the
 * greedy token to P->tok_out and advances S_dev to {token, pos + 1}.  NULL
 * when the variant is not instantiated. */
const void* lg_fused_variant(int layer_type, int out_type, int head_dim, int nrep);
int lg_fused_enqueue(const void* variant, const PkParams* P_dev, PkStep* S_dev, int n_layers, int nwg, hipStream_t s);
