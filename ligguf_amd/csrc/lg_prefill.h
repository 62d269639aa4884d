/* lg_prefill.h -- batched prefill (lg_prefill.hip), driven by the engine. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

/* Quantized activations of T tokens, structure of arrays (the GEMMs stage a
 * token tile with 16-byte loads).  Q8_K (Q4_K weights): qs [T][K] int8, d
 * [K/256][tld] block scales (tokens contiguous), bs [T][K/256][16] the
 * blocks' bsums.  Q8_0 (Q1_G weights): qs [T][K], d [K/32][tld] the fp16
 * block scales as floats, as [K/32][tld] the blocks' sums of q. */
struct PfQ8K {
    int8_t* qs;
    float* d;
    int16_t* bs;
    int* as;
    int tld;
};

/* one layer as the batched prefill reads it: fused Q|K|V and up|gate
 * matrices, all of the model's weight type (PfModel.wtype) */
struct PfLayer {
    const uint8_t *qkv, *ao, *ug, *down;
    uint32_t qkv_rsz, ao_rsz, ug_rsz, down_rsz;
    const float *att_norm, *ffn_norm, *q_norm, *k_norm;   /* q/k norms NULL for llama */
};

struct PfModel {
    const PfLayer* layers;   /* host array */
    int wtype;               /* LG_Q4_K (Q8_K activations) or LG_Q1_G (Q8_0) */
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
    PfQ8K q;         /* activations of width up to n_ff */
};

/* The layers of T prompt tokens at positions pos0.. (T <= B.tmax, tokens in
 * B.toks): KV rows pos0..pos0+T-1 written, B.x = the residual stream after
 * the last layer. */
int lg_prefill_layers(const PfModel& M, PfBuffers& B, int T, int pos0, hipStream_t s);

/* one Q4_K x Q8_K GEMM, out[t][r] (+)= sum_k W[r][k] x[t][k] over T tokens
 * of quantized activations (tests and benches) */
int lg_prefill_gemm_q4k(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out,
                        int ldo, int accumulate, hipStream_t s);
/* one Q1_G x Q8_0 GEMM, as lg_prefill_gemm_q4k */
int lg_prefill_gemm_q1g(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out,
                        int ldo, int accumulate, hipStream_t s);
/* rmsnorm (norm_w != NULL) and the activation quantizer of qtype (LG_Q8_K or
 * LG_Q8_0) for T tokens of width n */
int lg_prefill_quantize(int qtype, const float* x, int ldx, const float* norm_w, float eps, int n, int T,
                        const PfQ8K& q, hipStream_t s);
