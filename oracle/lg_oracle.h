/* lg_oracle.h -- CPU restatement of LiGGUF FAST's per-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker.  The
 * product (ligguf_amd/) never links or calls it.
 *
 * Arithmetic contract (what "the reference's algorithm" means here):
 *   - fp16 <-> fp32, weight dequantization and the activation quantizers are
 *     restated bit-exactly (the quantizers in their as-compiled -Ofast form);
 *   - every quantized dot product is split into the reference's exact integer
 *     sub-block sums, which the oracle computes in int64, and the floating
 *     combination of those integers, which the oracle evaluates in double and
 *     rounds once to float;
 *   - norms, RoPE, softmax, attention and SwiGLU are evaluated in double from
 *     float inputs and rounded once to float, except where the reference's
 *     own fp32 rounding is part of the semantics (the RoPE angle pos*freq is
 *     an fp32 product, the fp16 KV cache rounds k/v).
 * The reference evaluates the floating parts in fp32 in its own order, so
 * floating outputs agree with it to a tolerance, integer/byte outputs exactly.
 *
 * Pinning (tests/test_oracle.py): every function is checked against golden
 * vectors written by the reference engine built from its own sources
 * (tests/golden/), against the live reference build (oracle/_ref) when it is
 * present, and against closed forms / brute force where those exist.
 * or_sampler_topp (top-p / top-k sampling) has no golden vectors: closed
 * forms (greedy cases, tie order, a hand-made distribution with draws inside
 * each interval) and the live reference's sampler_topp pin it; the
 * reference's -Ofast sums make the two agree to float rounding of the
 * cumulative probabilities, not bit for bit.
 */
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gguf_type numbering, fast/lil_gguf.h:26-43 */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12,
    OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15, OR_Q1_0 = 40, OR_Q1_G = 41
};

/* Weight / model descriptors: same field order and meaning as lg_weight /
 * lg_layer_desc / lg_model_desc in include/ligguf_hip.h, so one host-side
 * description feeds both the oracle and the GPU engine. */
typedef struct {
    const void* data;   /* row-major rows of rsz bytes (wtensor, fast/lil_gguf.h:126-130) */
    int32_t type;       /* gguf_type */
    uint32_t rsz;       /* bytes per row (row_size, fast/lil_gguf.cpp:190-225) */
    int32_t rows;       /* output width d */
    int32_t cols;       /* input width n */
} or_weight;

typedef struct {
    const float* att_norm;
    or_weight att_q, att_k, att_v, att_out;
    const float* att_q_norm;
    const float* att_k_norm;
    const float* ffn_norm;
    or_weight ffn_up, ffn_down, ffn_gate;
} or_layer;

typedef struct {
    int32_t arch;       /* 0 = llama, 1 = qwen3 */
    int32_t n_layers, n_embed, n_heads, n_kv_heads, head_dim, kv_dim, n_ff, vocab_size, n_context, rope_dim;
    float rms_epsilon;
    const float* rope_freq;   /* rope_dim/2 entries (common.cpp:38-39) */
    or_weight token_embd, output;
    const float* output_norm;
    const or_layer* layers;
} or_model;

/* ---- A1: fp16 (fast/lil_math.cpp:37-86) ---- */
float or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
void or_f32_to_f16_row(const float* x, uint16_t* y, int64_t n);

/* ---- A3: dequantization (fast/lil_math.cpp:93-317) ---- */
int64_t or_row_size(int type, int64_t n);
int or_dequantize_row(int type, const void* x, float* y, int64_t n);

/* ---- A2: activation quantizers (fast/lil_math.cpp:329-394) ---- */
void or_quantize_q8_0(const float* x, int64_t n, void* y);   /* n % 32 == 0, y: n/32 x 34 B */
void or_quantize_q8_K(const float* x, int64_t n, void* y);   /* n % 256 == 0, y: n/256 x 292 B */

/* ---- A4/A5: quantized matvec (fast/lil_math.cpp:396-899) ----
 * xq: Q8_0 blocks for Q8_0/Q1_0/Q1_G weights, Q8_K blocks for Q2_K..Q6_K,
 *     fp32 vector for F32/F16 weights.
 * out[r] = row r . activation.  absout (optional) receives sum |terms| per
 * row, the scale for floating tolerances. */
int or_matvec_q(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, float* absout);
/* float activation in, quantized on the way as inference() does */
int or_matvec(int type, const void* w, uint32_t rsz, int n, int d, const float* x, float* out);

/* ---- A6/A7/A10 (fast/lil_math.cpp:901-937, fast/ligguf_fast_qk.cpp:119-123) ---- */
void or_rmsnorm(float* out, const float* x, const float* w, int n, float eps);
void or_rope(float* x, int n_heads, int head_dim, int rope_dim, int pos, const float* freq);
void or_swiglu(float* hb, const float* hb2, int n);

/* ---- A9: GQA decode attention (fast/ligguf_fast_qk.cpp:64-105) ----
 * kc/vc: fp16 rows [pos x kv_dim] for t < pos; k,v: fp32 current row. */
void or_attention(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                  int n_heads, int n_kv_heads, int head_dim, int pos, float* out);

/* ---- A12: whole per-token step (fast/ligguf_fast_qk.cpp:24-144) ---- */
typedef struct or_state or_state;
or_state* or_state_new(const or_model* m);
void or_state_free(or_state* s);
int or_state_pos(const or_state* s);
void or_state_set_pos(or_state* s, int pos);
/* inference(tok) at the state's position; copies logits (vocab floats) */
int or_inference(or_state* s, int tok, float* logits);
/* the next or_inference records the float vector before each activation
 * quantization into trace: [4*n_layers+1][max(n_embed, n_ff)] floats -- per
 * layer the rmsnorm'd attention input, the attention output, the rmsnorm'd
 * FFN input and the SwiGLU output, then the rmsnorm'd output-head input */
void or_state_trace(or_state* s, float* trace);
/* the next or_inference takes quantized activations from acts instead of
 * quantizing its own: at point k (numbered as in the trace) where forms[k]
 * is OR_Q8_K or OR_Q8_0, the matvecs whose weights read that form read the
 * blocks at acts + k*stride (block_q8_K / block_q8_0 layout; Q8_K bsums are
 * recomputed from the quants).  Each point of a step then starts from the
 * same quantized inputs as the step that recorded acts.  acts and forms must
 * outlive that call. */
void or_state_force(or_state* s, const void* acts, size_t stride, const int* forms);
/* fp16 KV rows of one layer for positions [p0, p0+np) */
void or_state_kv(const or_state* s, int layer, int p0, int np, uint16_t* k, uint16_t* v);
void or_state_kv_write(or_state* s, int layer, int p0, int np, const uint16_t* k, const uint16_t* v);
/* greedy argmax, first index wins ties (fast/ligguf_fast_qk.cpp:146-160) */
int or_argmax(const float* x, int n);
int or_sampler_topp(const float* logits, int n, float temp, float topp, int topk, float r01);

/* ---- (f)4: BERT embedding and vector-memory search (fast/vdb.cpp) ----
 * Descriptors laid out as lg_bert_layer_desc / lg_bert_desc
 * (include/ligguf_hip.h), bert_block / gguf_model's BERT fields
 * (fast/lil_gguf.h:146-160,200-205). */
typedef struct {
    or_weight attn_q, attn_k, attn_v, attn_out;
    const float *attn_q_bias, *attn_k_bias, *attn_v_bias, *attn_out_bias;
    const float *attn_norm_w, *attn_norm_b;
    or_weight ffn_up, ffn_down;
    const float *ffn_up_bias, *ffn_down_bias;
    const float *ffn_norm_w, *ffn_norm_b;
} or_bert_layer;

typedef struct {
    int32_t n_layers, n_embed, n_heads, n_ff, n_context, vocab_size, tok_cls, tok_sep;
    float eps;
    or_weight tok_embd, pos_embd, tok_types;
    const float *emb_norm_w, *emb_norm_b;
    const or_bert_layer* layers;
} or_bert;

/* layernorm (fast/lil_math.cpp:948-962) */
void or_layernorm(float* out, const float* x, const float* w, const float* b, int n, float eps);
/* bert_embed (fast/vdb.cpp:123-245) of bert_tokenize's ids: out[n_embed] */
int or_bert_embed(const or_bert* m, const int* toks, int ntok, float* out);
/* the same, recording the float vector at each of the 4 points per block
 * where matmul() would quantize it for a Q8_0/Q1 matrix -- the block input,
 * the attention output, the normalised attention-block output and the GELU
 * output -- into trace [n_layers][4][T][max(n_embed, n_ff)] (T = the
 * wrapped sequence length) */
int or_bert_embed_traced(const or_bert* m, const int* toks, int ntok, float* out, float* trace);
/* vdb_query's search (fast/vdb.cpp:352-368) over fp16 rows [n][dim]: the k
 * best at or above thr in the reference's insertion order; returns the count */
int or_vdb_search(const uint16_t* vecs, int n, int dim, const float* emb, float thr, int k, int* idx, float* sim);

#ifdef __cplusplus
}
#endif
