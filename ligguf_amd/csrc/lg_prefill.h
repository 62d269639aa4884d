/* lg_prefill.h -- batched prefill (lg_prefill.hip), driven by the engine. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

/* Quantized activations of T tokens, structure of arrays (the GEMMs stage a
 * token tile with 16-byte loads).  Q8_K form (K-quant weights): qs [T][K]
 * int8, d [K/256][tld] block scales (tokens contiguous), bs [T][K/256][16]
 * the blocks' bsums.  Q8_0 form (Q8_0, Q1_0, Q1_G weights): qs [T][K], d
 * [K/32][tld] the fp16 block scales as floats, as [K/32][tld] the blocks'
 * sums of q. */
struct PfQ8K {
    int8_t* qs;
    float* d;
    int16_t* bs;
    int* as;
    int tld;
    float* f;        /* F32 form (F32/F16 weights): the fp32 activations [T][K], nothing quantized */
};

/* one weight matrix as the prefill reads it: GGUF rows of `type` */
struct PfMat {
    const uint8_t* w;
    uint32_t rsz;
    int type;
    int rows;
};

/* one layer: Q|K|V as one stacked matrix (qkv_fused) or three, up|gate as
 * one (ug_fused) or two; each matrix of any type the batched GEMMs take */
struct PfLayer {
    PfMat q, k, v, qkv;
    PfMat ao, up, gate, ug, down;
    bool qkv_fused, ug_fused;
    const float *att_norm, *ffn_norm, *q_norm, *k_norm;   /* q/k norms NULL for llama */
};

struct PfModel {
    const PfLayer* layers;   /* host array */
    int n_layers, n_embed, n_heads, n_kv, head_dim, kv_dim, n_ff, n_ctx, rope_dim;
    float eps;
    const uint8_t* embd;
    uint32_t embd_rsz;
    int embd_t;
    const float* rope_freq;
    uint16_t* kc;
    uint16_t* vc;
};

/* device buffers for up to tmax tokens per pass */
struct PfBuffers {
    int tmax;
    int* toks;       /* [tmax] */
    float* x;        /* [tmax][n_embed] residual stream */
    float* qkv;      /* [tmax][n_embed + 2 kv_dim] */
    float* att;      /* [tmax][n_embed] */
    float* ug;       /* [tmax][2 n_ff] */
    PfQ8K qk;        /* Q8_K form, width up to n_ff (qs NULL when no matrix takes it) */
    PfQ8K q0;        /* Q8_0 form (likewise) */
    PfQ8K qf;        /* F32 form (likewise; only f and tld) */
    /* activation trace of one pass (NULL: none): token t's activation k in
     * block_q8_K / block_q8_0 rows at trace + (t (4 L + 1) + k) stride */
    uint8_t* trace;
    size_t trace_stride;
};

/* activation form a weight type takes: LG_Q8_K, LG_Q8_0, LG_F32 (F32/F16
 * weights), or -1 when the batched GEMMs do not take the type */
int lg_prefill_act_type(int wtype);

/* the prefill attention's head widths and query heads per KV head */
int lg_prefill_attn_supported(int head_dim, int nrep);

/* The layers of T prompt tokens at positions pos0.. (T <= B.tmax, tokens in
 * B.toks): KV rows pos0..pos0+T-1 written, B.x = the residual stream after
 * the last layer. */
int lg_prefill_layers(const PfModel& M, PfBuffers& B, int T, int pos0, hipStream_t s);

/* One GEMM out[t][r] (+)= sum_k W[r][k] x[t][k] over T tokens of activations
 * quantized in the form lg_prefill_act_type(wtype) gives (tests, benches and
 * the layer passes). */
int lg_prefill_gemm(int wtype, const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out,
                    int ldo, int accumulate, hipStream_t s);
/* LG_PF_GEMM16=1 in the environment: the 16 x 16 int8-MFMA kernels (they
 * read regrouped Q8_0 / Q1_0 rows, Q6_K and Q1_G from the GGUF rows only) */
bool lg_prefill_gemm16();
/* rmsnorm (norm_w != NULL) and the activation quantizer of qtype (LG_Q8_K,
 * n a multiple of 256, or LG_Q8_0, n a multiple of 32; LG_F32: the fp32
 * values into q.f) for T tokens of width n */
int lg_prefill_quantize(int qtype, const float* x, int ldx, const float* norm_w, float eps, int n, int T,
                        const PfQ8K& q, hipStream_t s);

/* F32/F16 weights x fp32 activations on fp32 MFMA (lg_bert.hip's token
 * GEMM): out[t][r] (+)= W[r] . x[t] */
int lg_fgemm_tokens(int wtype, const uint8_t* W, int rows, int cols, const float* x, int ldx, int T, float* out, int ldo,
                    int accumulate, hipStream_t s);
