/* C-ABI harness around the reference LiGGUF FAST engine, compiled from the
 * reference's own unmodified sources (see oracle/Makefile).  TEST
 * INFRASTRUCTURE ONLY: it is the checker and the CPU baseline, never part of
 * the product path.
 *
 * Every entry point forwards to the reference function it names:
 *   fp1632_init / fp16_to_fp32 / f32_to_f16_row   fast/lil_math.cpp:37-86
 *   dequantize_row                                fast/lil_math.cpp:300-317
 *   quantize_q8_0 / quantize_q8_K                 fast/lil_math.cpp:329-394
 *   matmul / matmul2 / matmul3                    fast/lil_math.cpp:748-899
 *   rope / rmsnorm / rmsnorm_inplace / softmax    fast/lil_math.cpp:901-976
 *   inference()                                   fast/ligguf_fast_qk.cpp:24-144
 *   save_model_state / load_model_state           fast/ligguf_fast_qk.cpp:216-302
 *   model_state::allocate                         fast/common.cpp:11-40
 *   gguf_model::open_mmap/read_gguf/read_tokenizer fast/lil_gguf.cpp:227-395
 * The attention entry (ref_attention) replays the inline attention block of
 * inference() (fast/ligguf_fast_qk.cpp:64-105) on caller buffers, calling the
 * reference's own vec_dot_f32 / vec_dot_f16_f32 / softmax / fp16 LUT.
 */
#include <stdint.h>
#include <string.h>
#include <algorithm>
#include <vector>
#include <string>
#include "common.h"
#include "lil_gguf.h"
#include "lil_math.h"

extern void inference(int tok);
extern bool load_model_state(const char* fn);
extern bool save_model_state(const char* fn);
extern int sampler_greedy();
extern int sampler_topp();

extern "C" {

void ref_init(void) { fp1632_init(); }

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }

void ref_f32_to_f16_row(const float* x, uint16_t* y, int n) { f32_to_f16_row(x, y, n); }

void ref_f16_to_f32_row(const uint16_t* x, float* y, int n)
{
    for (int i = 0; i < n; i++) y[i] = fp16_to_fp32(x[i]);
}

void ref_dequantize_row(int type, const void* in, float* out, int64_t n)
{
    dequantize_row((gguf_type)type, in, out, n);
}

/* y receives n/32 block_q8_0 (34 B each) */
void ref_quantize_q8_0(const float* x, int n, void* y)
{
    ftensor xv(x, x + n);
    qtensor q(n / QK8_0);
    quantize_q8_0(q, xv);
    memcpy(y, q.data(), (size_t)(n / QK8_0) * sizeof(block_q8_0));
}

/* y receives n/256 block_q8_K (292 B each); n must be a multiple of 256 */
void ref_quantize_q8_K(const float* x, int n, void* y)
{
    ftensor xv(x, x + n);
    ktensor q(n / QK_K);
    quantize_q8_K(q, xv);
    memcpy(y, q.data(), (size_t)(n / QK_K) * sizeof(block_q8_K));
}

static bool is_q8_0_family(int t) { return t == Q8_0 || t == Q1_0 || t == Q1_G; }

/* One weight matrix times a float activation, the way inference() drives it:
 * Q8_0/Q1 weights quantize the activation to Q8_0 inside matmul(), every other
 * quantized type gets a quantize_q8_K first (fast/ligguf_fast_qk.cpp:39-40). */
void ref_matmul(int type, const void* w, uint32_t rsz, int n, int d, const float* x, float* out)
{
    ftensor src(x, x + n), o(d);
    wtensor wt; wt.ptr = (uint8_t*)w; wt.type = (gguf_type)type; wt.rsz = rsz;
    if (is_q8_0_family(type) || type == F32 || type == F16) {
        matmul(o, &src, NULL, NULL, wt, n, d);
    } else {
        ktensor xq(n / QK_K);
        quantize_q8_K(xq, src);
        matmul(o, &src, &xq, NULL, wt, n, d);
    }
    memcpy(out, o.data(), (size_t)d * sizeof(float));
}

/* matmul() with a caller-supplied pre-quantized activation (Q8_K blocks for
 * K-quant weights, Q8_0 blocks for Q8_0/Q1 weights). */
void ref_matmul_q(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out)
{
    ftensor o(d);
    wtensor wt; wt.ptr = (uint8_t*)w; wt.type = (gguf_type)type; wt.rsz = rsz;
    if (is_q8_0_family(type)) {
        const block_q8_0* b = (const block_q8_0*)xq;
        qtensor q(b, b + n / QK8_0);
        matmul(o, NULL, NULL, &q, wt, n, d);
    } else {
        const block_q8_K* b = (const block_q8_K*)xq;
        ktensor q(b, b + n / QK_K);
        matmul(o, NULL, &q, NULL, wt, n, d);
    }
    memcpy(out, o.data(), (size_t)d * sizeof(float));
}

void ref_rmsnorm(float* out, const float* x, const float* w, int n, float eps)
{
    ftensor xv(x, x + n), o(n);
    rmsnorm(o, xv, (float*)w, n, eps);
    memcpy(out, o.data(), (size_t)n * sizeof(float));
}

void ref_rmsnorm_inplace(float* x, const float* w, int n, float eps)
{
    rmsnorm_inplace(x, (float*)w, n, eps);
}

void ref_softmax(float* x, int n) { softmax(x, n); }

void ref_rope(float* x, int n_heads, int head_dim, int rope_dim, int pos, const float* freq, int n_freq)
{
    gguf_model mdl;
    mdl.head_dim = head_dim;
    mdl.rope_dim = rope_dim;
    ftensor xv(x, x + (size_t)n_heads * head_dim);
    ftensor fv(freq, freq + n_freq);
    rope(xv, n_heads, pos, mdl, fv);
    memcpy(x, xv.data(), xv.size() * sizeof(float));
}

/* rope_freq table exactly as model_state::allocate() builds it (common.cpp:38-39) */
void ref_rope_freq(float base, int rope_dim, float* out)
{
    for (int i = 0; i < rope_dim / 2; i++) out[i] = powf(base, -2.0f * (float)i / (float)rope_dim);
}

/* The attention block of inference() for one layer, on caller buffers:
 * q [n_heads*hd] fp32 (already normed/roped), k,v [kv_dim] fp32 for position
 * pos, kc/vc fp16 rows [(pos+1) x kv_dim] (row pos is ignored: the fp32 k/v
 * are used for t == pos, as at fast/ligguf_fast_qk.cpp:77-79,98-99).
 * out [n_heads*hd].  att is scratch [n_heads*(pos+1)]. */
void ref_attention(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, float* att_scratch)
{
    const float att_scale = 1.0f / sqrtf(head_dim);
    const int kv_dim = n_kv_heads * head_dim;
    const int nrep = n_heads / n_kv_heads;
    const int ctx = pos + 1;

    MULTITHREAD
    for (int h = 0; h < n_heads; h++) {
        float* att = att_scratch + (size_t)h * ctx;
        const float* qh = q + h * head_dim;
        const float* kh = k + (h / nrep) * head_dim;
        const float* vh = v + (h / nrep) * head_dim;
        for (int t = 0; t <= pos; t++) {
            float score;
            if (t == pos) score = vec_dot_f32(qh, kh, head_dim);
            else score = vec_dot_f16_f32(kc + (size_t)t * kv_dim + (h / nrep) * head_dim, qh, head_dim);
            att[t] = score * att_scale;
        }
        softmax(att, pos + 1);
        float* xb = out + h * head_dim;
        memset(xb, 0, head_dim * sizeof(float));
        for (int t = 0; t <= pos; t++) {
            float a = att[t];
            if (t == pos) {
                for (int i = 0; i < head_dim; i++) xb[i] += a * vh[i];
            } else {
                const uint16_t* vr = vc + (size_t)t * kv_dim + (h / nrep) * head_dim;
                for (int i = 0; i < head_dim; i++) xb[i] += a * fp16_to_fp32(vr[i]);
            }
        }
    }
}

/* ---- whole engine (global g_m, as in the reference driver) ---- */

/* Open a GGUF through the reference loader and allocate the state, as main()
 * does (fast/ligguf_fast_qk.cpp:572-575). n_ctx > 0 overrides the context. */
int ref_model_open(const char* path, int n_ctx)
{
    /* read_gguf() adds to the tensor and metadata maps without clearing them
     * (fast/lil_gguf.cpp:357-372): a second open in one process must start
     * from empty maps, as the reference's single-model process does, or
     * read_llama would bind the previous file's stale tensors.  The KV cache
     * is cleared for the same reason (allocate() keeps old contents). */
    g_m.m.close_mmap();
    g_m.m.tensors.clear();
    g_m.m.meta_kv.clear();
    std::fill(g_m.kc.begin(), g_m.kc.end(), (uint16_t)0);
    std::fill(g_m.vc.begin(), g_m.vc.end(), (uint16_t)0);
    g_m.pos = 0;
    g_m.u_context = n_ctx;
    if (!g_m.m.open_mmap(path)) return -1;
    if (!g_m.m.read_gguf()) return -2;
    g_m.allocate();
    if (!g_m.m.read_tokenizer()) return -3;
    return 0;
}

/* Describe a model that already sits in host memory (no GGUF file): the
 * tensors are bound straight into g_m.m like read_llama/read_qwen3 bind mmap
 * pointers (fast/lil_gguf.cpp:397-499). */
struct ref_weight { const void* ptr; int32_t type; uint32_t rsz; };
struct ref_layer {
    const float* att_norm; ref_weight att_q, att_k, att_v, att_out;
    const float* att_q_norm; const float* att_k_norm; const float* ffn_norm;
    ref_weight ffn_up, ffn_down, ffn_gate;
};
struct ref_model {
    int32_t qwen3; int32_t n_layers, n_embed, n_heads, n_kv_heads, head_dim, kv_dim, n_ff, vocab_size, n_context, rope_dim;
    float rms_epsilon; float rope_base;
    ref_weight embed, output; const float* output_norm; const ref_layer* layers;
};

static wtensor mkw(const ref_weight& w)
{
    wtensor r; r.ptr = (uint8_t*)w.ptr; r.type = (gguf_type)w.type; r.rsz = w.rsz; return r;
}

int ref_model_bind(const ref_model* d)
{
    gguf_model& m = g_m.m;
    m.arch = d->qwen3 ? "qwen3" : "llama";
    m.n_layers = d->n_layers; m.n_embed = d->n_embed; m.n_heads = d->n_heads; m.n_kv_heads = d->n_kv_heads;
    m.head_dim = d->head_dim; m.kv_dim = d->kv_dim; m.n_ff = d->n_ff; m.vocab_size = d->vocab_size;
    m.n_context = d->n_context; m.rope_dim = d->rope_dim; m.rms_epsilon = d->rms_epsilon; m.rope_base = d->rope_base;
    m.tok_eos = -1;
    m.t_embed = mkw(d->embed); m.t_out = mkw(d->output); m.t_outnorm = (float*)d->output_norm;
    m.tr.resize(d->n_layers);
    for (int l = 0; l < d->n_layers; l++) {
        const ref_layer& s = d->layers[l];
        trans_block& t = m.tr[l];
        t.att_norm = (float*)s.att_norm; t.att_q = mkw(s.att_q); t.att_k = mkw(s.att_k); t.att_v = mkw(s.att_v);
        t.att_out = mkw(s.att_out); t.att_q_norm = (float*)s.att_q_norm; t.att_k_norm = (float*)s.att_k_norm;
        t.ffn_norm = (float*)s.ffn_norm; t.ffn_up = mkw(s.ffn_up); t.ffn_down = mkw(s.ffn_down); t.ffn_gate = mkw(s.ffn_gate);
    }
    g_m.u_context = 0;
    g_m.pos = 0;
    g_m.allocate();
    return 0;
}

void ref_model_info(int32_t* o)
{
    const gguf_model& m = g_m.m;
    o[0] = m.n_layers; o[1] = m.n_embed; o[2] = m.n_heads; o[3] = m.n_kv_heads; o[4] = m.head_dim;
    o[5] = m.kv_dim; o[6] = m.n_ff; o[7] = m.vocab_size; o[8] = m.n_context; o[9] = m.rope_dim;
    o[10] = m.arch == "qwen3"; o[11] = m.tok_eos; o[12] = g_m.pos;
}

const float* ref_rope_freq_table(void) { return g_m.rope_freq.data(); }

/* inference(tok) at the current g_m.pos; copies the logits out when non-NULL */
void ref_inference(int tok, float* logits)
{
    inference(tok);
    if (logits) memcpy(logits, g_m.logits.data(), g_m.logits.size() * sizeof(float));
}

int ref_get_pos(void) { return g_m.pos; }
void ref_set_pos(int pos) { g_m.pos = pos; }

/* fp16 K/V cache rows of one layer for positions [p0, p0+np) */
void ref_kv_rows(int layer, int p0, int np, uint16_t* k, uint16_t* v)
{
    const size_t loff = (size_t)layer * g_m.m.n_context * g_m.m.kv_dim;
    const size_t off = loff + (size_t)p0 * g_m.m.kv_dim;
    const size_t cnt = (size_t)np * g_m.m.kv_dim;
    if (k) memcpy(k, g_m.kc.data() + off, cnt * sizeof(uint16_t));
    if (v) memcpy(v, g_m.vc.data() + off, cnt * sizeof(uint16_t));
}

void ref_kv_write_rows(int layer, int p0, int np, const uint16_t* k, const uint16_t* v)
{
    const size_t loff = (size_t)layer * g_m.m.n_context * g_m.m.kv_dim;
    const size_t off = loff + (size_t)p0 * g_m.m.kv_dim;
    const size_t cnt = (size_t)np * g_m.m.kv_dim;
    if (k) memcpy(g_m.kc.data() + off, k, cnt * sizeof(uint16_t));
    if (v) memcpy(g_m.vc.data() + off, v, cnt * sizeof(uint16_t));
}

/* greedy argmax over the current logits, first index wins (fast/ligguf_fast_qk.cpp:146-160) */
int ref_sampler_greedy(void)
{
    return sampler_greedy();
}

/* sampler_topp (fast/ligguf_fast_qk.cpp:172-214) over n given logits with
 * srand(seed) before it; the model state's logits, vocabulary size, sampler
 * settings and work buffer are restored afterwards */
int ref_sampler_topp(const float* logits, int n, float temp, float topp, int topk, unsigned seed)
{
    std::vector<float> keep_logits(n);
    keep_logits.swap(g_m.logits);
    g_m.logits.assign(logits, logits + n);
    const int keep_vocab = g_m.m.vocab_size;
    const int keep_topk = g_m.topk;
    const float keep_topp = g_m.topp, keep_temp = g_m.temp;
    std::vector<sampler_entry> keep_samp(n);
    keep_samp.swap(g_m.samp);
    g_m.m.vocab_size = n;
    g_m.temp = temp;
    g_m.topp = topp;
    g_m.topk = topk;
    srand(seed);
    const int tok = sampler_topp();
    g_m.logits.swap(keep_logits);
    g_m.samp.swap(keep_samp);
    g_m.m.vocab_size = keep_vocab;
    g_m.topk = keep_topk;
    g_m.topp = keep_topp;
    g_m.temp = keep_temp;
    return tok;
}

/* save_model_state / load_model_state (fast/ligguf_fast_qk.cpp:216-302) on g_m */
int ref_state_save(const char* fn) { return save_model_state(fn) ? 0 : -1; }
int ref_state_load(const char* fn) { return load_model_state(fn) ? 0 : -1; }

/* the current logits (vocab floats) */
void ref_logits(float* out) { memcpy(out, g_m.logits.data(), g_m.logits.size() * sizeof(float)); }

void ref_model_close(void)
{
    g_m.m.close_mmap();
}

} /* extern "C" */
