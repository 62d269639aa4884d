/* ligguf_hip.h -- C-ABI of the gfx950 (MI355X) decode path of LiGGUF FAST.
 *
 * libligguf_hip.so replaces the hot paths of the reference's math layer
 * (fast/lil_math.h:5-39, fast/lil_math.cpp, fast/arch_avx2.h) and the inline
 * per-token sequence of inference() (fast/ligguf_fast_qk.cpp:24-144).  The
 * reference's host code -- GGUF loader, tokenizer, samplers, chat and state
 * save -- keeps running on the CPU and calls this layer at model upload, per
 * step and for KV state I/O.
 *
 * Conventions
 *   - Every entry point returns LG_OK (0) or a negative LG_ERR_* code and
 *     never aborts (the reference aborts on unsupported types,
 *     fast/lil_math.cpp:313-315,771-773, and asserts shapes, :360,752,903).
 *     The message of the last failure is lg_last_error(ctx), or
 *     lg_last_error(NULL) for the per-op calls, which keep it per host thread.
 *   - Weight type codes are the reference's gguf_type values
 *     (fast/lil_gguf.h:26-43).  Block layouts are the GGUF ones
 *     (fast/lil_gguf.h:64-119): weights are consumed as stored, rows of rsz
 *     bytes (wtensor, fast/lil_gguf.h:126-130).
 *   - Per-op calls take device pointers and a HIP stream passed as void*
 *     (NULL = the default stream); they are asynchronous.
 *   - A context owns one device, one stream and the uploaded model; it is not
 *     thread-safe (the reference's op layer is not reentrant either: global
 *     g_m and the static m_xq8, fast/lil_math.cpp:13).
 */
#ifndef LIGGUF_HIP_H
#define LIGGUF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define LG_OK 0
#define LG_ERR_ARG (-1)      /* bad argument, shape or size */
#define LG_ERR_TYPE (-2)     /* unsupported tensor type */
#define LG_ERR_HIP (-3)      /* HIP runtime error */
#define LG_ERR_STATE (-4)    /* call out of order (no model, context full ...) */
#define LG_ERR_NOMEM (-5)    /* device allocation failed */

/* ---- tensor types: gguf_type (fast/lil_gguf.h:26-43) ---- */
enum lg_type {
    LG_F32 = 0, LG_F16 = 1, LG_Q8_0 = 8, LG_Q2_K = 10, LG_Q3_K = 11, LG_Q4_K = 12,
    LG_Q5_K = 13, LG_Q6_K = 14, LG_Q8_K = 15, LG_Q1_0 = 40, LG_Q1_G = 41
};

enum lg_arch { LG_ARCH_LLAMA = 0, LG_ARCH_QWEN3 = 1 };

/* Bytes of one row of n values of type t (row_size, fast/lil_gguf.cpp:190-225),
 * or -1 when n does not fit the block size.  Q8_K is the activation format
 * (block_q8_K, fast/lil_gguf.h:115-119). */
int64_t lg_row_size(int type, int64_t n);

/* ===================================================================== */
/* Context and model                                                      */
/* ===================================================================== */
typedef struct lg_ctx lg_ctx;

/* Open device `device` (HIP ordinal).  Replaces nothing in the reference,
 * whose state is the global model_state g_m (fast/common.h:33-72). */
int lg_create(int device, lg_ctx** out);
int lg_destroy(lg_ctx* ctx);
const char* lg_last_error(const lg_ctx* ctx);

/* One weight matrix in host memory: the reference's wtensor
 * {ptr, type, rsz} (fast/lil_gguf.h:126-130) plus its shape. */
typedef struct {
    const void* data;   /* host pointer to rows * rsz bytes */
    int32_t type;       /* lg_type */
    uint32_t rsz;       /* bytes per row */
    int32_t rows;       /* output width d */
    int32_t cols;       /* input width n */
} lg_weight;

/* One transformer block: trans_block (fast/lil_gguf.h:132-144).  Norm
 * vectors are F32 host arrays (n_embed, or head_dim for the Qwen3 QK norms). */
typedef struct {
    const float* att_norm;
    lg_weight att_q, att_k, att_v, att_out;
    const float* att_q_norm;    /* qwen3 only */
    const float* att_k_norm;    /* qwen3 only */
    const float* ffn_norm;
    lg_weight ffn_up, ffn_down, ffn_gate;
} lg_layer_desc;

/* The model: the fields of gguf_model the decode path reads
 * (fast/lil_gguf.h:161-219) plus the host RoPE table of
 * model_state::allocate (fast/common.cpp:38-39), uploaded as is so the
 * device uses bit-identical frequencies. */
typedef struct {
    int32_t arch;               /* lg_arch */
    int32_t n_layers, n_embed, n_heads, n_kv_heads, head_dim, kv_dim, n_ff, vocab_size, n_context, rope_dim;
    float rms_epsilon;
    const float* rope_freq;     /* rope_dim/2 floats */
    lg_weight token_embd, output;
    const float* output_norm;
    const lg_layer_desc* layers;  /* n_layers entries */
} lg_model_desc;

/* Copy the model into HBM (weights, norms, RoPE table) and allocate the fp16
 * KV cache [n_layers][n_context][kv_dim] (fast/common.cpp:31-32) plus the
 * activation buffers.  The host memory can be released afterwards. */
int lg_load_model(lg_ctx* ctx, const lg_model_desc* desc);

/* inference(tok) at position pos (fast/ligguf_fast_qk.cpp:24-144): the whole
 * layer loop on the device, KV row pos written, logits[vocab] copied to
 * logits_host when it is not NULL.  Synchronous on return. */
int lg_decode_step(lg_ctx* ctx, int tok, int pos, float* logits_host);

/* Same as lg_decode_step but leaves the logits on the device (returned via
 * lg_logits_device) and does not wait: the caller synchronises with
 * lg_sync.  Lets a driver keep the decode loop free of host round trips. */
int lg_decode_step_async(lg_ctx* ctx, int tok, int pos);
int lg_sync(lg_ctx* ctx);
const float* lg_logits_device(lg_ctx* ctx);

/* Which implementation runs the decode step.  LG_PATH_FUSED is five fused
 * kernels per layer (rmsnorm+QKV, attention with its merge, att_out +
 * residual, rmsnorm + up|gate + SwiGLU, down + residual) and one for the
 * output head and greedy argmax, replayed from a HIP graph captured on first
 * use (set LG_NO_GRAPH=1 in the environment before lg_create to launch them
 * directly); token and position live in device memory, so consecutive greedy
 * steps need no host-to-device copy.  LG_PATH_PERSISTENT is the same phases in
 * one cooperative kernel per token with flag syncs between them.
 * LG_PATH_MULTI is one kernel per operation and serves every model.  AUTO
 * (the default) takes FUSED when the model has an instantiation, else MULTI.
 * FUSED needs one layer type for the layer matrices (Q4_K or Q5_K layers
 * may also carry Q5_K / Q6_K attn_v and ffn_down matrices in any layer, as
 * Q4_K_M / Q4_K_S / Q5_K_M files do) with a matching output type and
 * head_dim 128, 64 or 48 in one of the width classes the library is built
 * with: n_embed 4096 with n_ff 12288 (Q2_K..Q6_K, Q1_G, Q1_0, Q8_0 layers; 1,
 * 4 or 8 query heads per KV head) or 14336 (Q4_K, Q8_0; 4),
 * 2560 / 9728 (Q4_K; 4), 2048 / 5632 (Q4_K, Q8_0; head_dim 64, 8), and any
 * widths up to 2048 / 2048 (Q8_0 with head_dim 48 or 64, Q4_K with 64; one
 * query head per KV head) -- widths are runtime values within a class.
 * FUSED reads Q8_0 / Q6_K / Q3_K / Q1_0 / Q1_G matrices (the output head, uniform
 * layers of those types, a mixed layer's Q6_K attn_v / ffn_down) from copies
 * regrouped for aligned loads, which costs their size again in device
 * memory; LG_NO_REGROUP=1 in the environment before lg_create reads the GGUF
 * rows instead (same results).  PERSISTENT is instantiated for n_embed 4096
 * / n_ff 12288 with one type for every layer matrix.  Both
 * compute the reference's inference() sequence with the same quantizers and
 * dot decompositions.  No counterpart in the reference (one CPU engine). */
#define LG_PATH_AUTO 0
#define LG_PATH_PERSISTENT 1
#define LG_PATH_MULTI 2
#define LG_PATH_FUSED 3
int lg_set_decode_path(lg_ctx* ctx, int path);
/* the path the next step takes (LG_PATH_FUSED, LG_PATH_PERSISTENT or LG_PATH_MULTI), -1 without a model */
int lg_decode_path(const lg_ctx* ctx);

/* Phase tracing of the fused and persistent steps (no counterpart in the reference,
 * whose only instrumentation is wall-clock per token,
 * fast/ligguf_fast_qk.cpp:316-331).  lg_trace_size(ctx) bytes of device
 * memory at trace_dev receive, for the NEXT fused or persistent step only, four
 * 100 MHz timestamps per phase and workgroup -- [5*n_layers+1][nwg][4]:
 * phase entry, dependency wait over, activation built, phase published.
 * (for the fused kernels: entry, loads issued, activation built, done).
 * lg_trace_size is 0 when the model runs on the multi-kernel path. */
int lg_trace_next_step(lg_ctx* ctx, uint64_t* trace_dev);
size_t lg_trace_size(const lg_ctx* ctx);

/* Activation trace of the NEXT decode step on any path (no counterpart in
 * the reference; for parity tests): lg_trace_acts_size(ctx) bytes of device
 * memory at trace_dev receive every quantized activation the step builds, in
 * slots of lg_trace_acts_size(ctx) / (4*n_layers + 1) bytes -- per layer the
 * attention input (rmsnorm), the attention output, the FFN input (rmsnorm)
 * and the SwiGLU output, then the output head's input -- each in the GGUF
 * block layout of the activation its weights read (block_q8_K when that is
 * a K-quant, block_q8_0 for Q8_0/Q1_0/Q1_G; fast/lil_gguf.h:64-67,115-119),
 * i.e. the quantize_q8_K / quantize_q8_0 outputs of inference()
 * (fast/ligguf_fast_qk.cpp:39,108,116,126,140). */
int lg_trace_acts_next_step(lg_ctx* ctx, void* trace_dev);
size_t lg_trace_acts_size(const lg_ctx* ctx);
/* The same for every token of the NEXT lg_prefill when it runs batched (no
 * counterpart in the reference; for parity tests): n * lg_trace_acts_size
 * bytes at trace_dev, token t's slots at t * lg_trace_acts_size, the output
 * head's input for the last token only.  A prompt that runs token by token
 * drops the request. */
int lg_trace_acts_next_prefill(lg_ctx* ctx, void* trace_dev);

/* Times one kernel of the fused step (no counterpart in the reference; for
 * benchmarks and profiles): phase 0 rmsnorm + QKV, 1 attention, 2 att_out,
 * 3 rmsnorm + up|gate + SwiGLU, 4 down, 5 output head + argmax, launched
 * `iters` times directly on the context's stream at layers layer0,
 * layer0 + 1, ... (mod n_layers), between two HIP events; *avg_us receives
 * the mean time per launch.  The kernels work on the device state of the
 * last step (run and synchronize one first); the next step rewrites
 * everything they touch.  LG_ERR_STATE unless the fused path is in use. */
int lg_time_fused_phase(lg_ctx* ctx, int phase, int layer0, int iters, float* avg_us);

/* HBM read probe (no counterpart in the reference; the practical read
 * bound for benchmarks): reads the `bytes` bytes at buf (device memory,
 * 16-byte aligned, a multiple of 16) once per pass, `iters` timed passes
 * after an untimed one on `stream` (NULL: the null stream); *avg_us
 * receives the mean time per pass.  Writes nothing. */
int lg_hbm_read_probe(const void* buf, size_t bytes, int iters, float* avg_us, void* stream);

/* Greedy argmax of the current device logits, first index wins ties
 * (sampler_greedy, fast/ligguf_fast_qk.cpp:146-160). */
int lg_argmax(lg_ctx* ctx, int* tok_out);

/* n greedy decode steps queued back to back: the step at position pos takes
 * token tok, each later one the greedy token of the step before it, which
 * stays on the device (no host round trip per token on the fused and
 * persistent paths); toks_out[i] is the greedy token of step pos + i.  The
 * same tokens, logits and KV rows as n rounds of lg_decode_step + lg_argmax
 * -- the reference's generation loop feeding sampler_greedy's token back to
 * inference() (fast/ligguf_fast_qk.cpp:368-382) -- except that it does not
 * stop at an end-of-sequence token: the caller truncates toks_out there.
 * Needs pos + n <= n_context; the device logits are the last step's.  No
 * counterpart in the reference (its loop runs on the host). */
int lg_decode_greedy(lg_ctx* ctx, int tok, int pos, int n, int* toks_out);

/* Top-p / top-k sampling of the current device logits (sampler_topp,
 * fast/ligguf_fast_qk.cpp:172-214, with g_m.temp, g_m.topp, g_m.topk as
 * arguments): softmax at temperature temp, entries by probability descending
 * (ties: lower token first), the cutoff where the cumulative probability
 * reaches topp (topp <= 0: the first entry's; above 1: 1) or topk entries
 * (topk <= 0: all), then the entry where it reaches r01 times the cutoff's.
 * r01 is the caller's uniform draw in [0, 1] -- the reference's
 * (float)rand() / (float)RAND_MAX.  temp <= 0 gives lg_argmax's token.
 * The first call allocates a workspace of about 9 bytes per vocabulary entry
 * and one pinned host word; vocabularies above 2^21 entries are refused
 * (LG_ERR_ARG).  LG_ERR_STATE if a workgroup's bounded publish wait expired.
 * Synchronous. */
int lg_sample_topp(lg_ctx* ctx, float temp, float topp, int topk, float r01, int* tok_out);

/* lg_sample_topp over n device floats at logits_dev (no context): a helper
 * for tests and benchmarks -- it allocates and frees its workspace (about
 * 9 n bytes) on every call and runs on the null stream, waiting for it.
 * Decode loops use lg_sample_topp, whose workspace lives in the context. */
int lg_sample_topp_device(const float* logits_dev, int n, float temp, float topp, int topk, float r01, int* tok_out);

/* feed_text's prompt loop (fast/ligguf_fast_qk.cpp:340-356): n tokens at
 * positions pos0..pos0+n-1, equal to n sequential lg_decode_step calls;
 * logits of the last token to logits_host (NULL allowed). */
int lg_prefill(lg_ctx* ctx, const int* toks, int n, int pos0, float* logits_host);

/* How lg_prefill runs a prompt (no counterpart in the reference, which
 * feeds it token by token).  BATCHED: layer passes over up to 512 tokens,
 * each weight matrix read once per pass and multiplied by all of them with
 * int8 MFMA GEMMs, the tokens' integer sub-block sums and quantizers those
 * of the step; the logits then match n sequential steps to fp32 rounding (an
 * int8 rounding of an activation may differ in rare tokens).  Takes every
 * layer type -- Q2_K..Q6_K, Q8_0, Q1_0, Q1_G on int8 MFMA, F32/F16 on fp32
 * MFMA, in any mix (a Q4_K_M-style model with Q6_K matrices among its Q4_K
 * ones included) -- and needs head_dim 48, 64 or 128 with 1, 2, 4 or 8 query
 * heads per KV head.  STEPS: one
 * decode step per token, bit-equal to n lg_decode_step calls.  AUTO (the
 * default): BATCHED when the model allows it and n >= 2, else STEPS.
 * lg_prefill_path reports what a prompt of 2+ tokens takes (-1 without a
 * model). */
#define LG_PREFILL_AUTO 0
#define LG_PREFILL_STEPS 1
#define LG_PREFILL_BATCHED 2
int lg_set_prefill_path(lg_ctx* ctx, int path);
int lg_prefill_path(const lg_ctx* ctx);

/* fp16 KV rows [pos0, pos0+npos) of layers [layer0, layer0+nlayers) to/from
 * host arrays laid out [nlayers][npos][kv_dim] -- the per-layer blocks of the
 * reference's state file (save/load_model_state,
 * fast/ligguf_fast_qk.cpp:216-302). */
int lg_kv_read(lg_ctx* ctx, int layer0, int nlayers, int pos0, int npos, uint16_t* k_host, uint16_t* v_host);
int lg_kv_write(lg_ctx* ctx, int layer0, int nlayers, int pos0, int npos, const uint16_t* k_host,
                const uint16_t* v_host);

/* The reference's state file (save_model_state / load_model_state,
 * fast/ligguf_fast_qk.cpp:216-302): the 24-byte packed model_file header
 * {int pos; int n_context; uint64 kv_size; uint64 logits_size}
 * (fast/common.h:26-31), per layer the first pos x kv_dim fp16 K values,
 * then the same for V, then vocab fp32 logits.  lg_state_save writes the
 * device cache rows [0, pos) and the logits of the last step (the reference
 * refuses pos 0); lg_state_load checks the header as the reference does
 * (kv_size = n_layers x pos x kv_dim, logits_size = vocab) and pos against
 * this context, fills the device cache and logits, and returns pos, at which
 * the next step continues (and the logits, when logits_host is not NULL).
 * Files are interchangeable with the reference's own. */
int lg_state_save(lg_ctx* ctx, const char* path, int pos);
int lg_state_load(lg_ctx* ctx, const char* path, int* pos_out, float* logits_host);

/* ===================================================================== */
/* Per-op entry points (device pointers, asynchronous on `stream`)        */
/* ===================================================================== */

/* dequantize_row (fast/lil_math.cpp:300-317): n values of `type` at x to
 * fp32 y; bit-identical to the reference. */
int lg_dequantize_row(int type, const void* x, float* y, int64_t n, void* stream);

/* quantize_q8_0 (fast/lil_math.cpp:329-351): n % 32 == 0, y gets n/32 blocks
 * of 34 B; bit-identical to the reference as compiled. */
int lg_quantize_q8_0(const float* x, int64_t n, void* y, void* stream);

/* quantize_q8_K (fast/lil_math.cpp:358-394): n % 256 == 0, y gets n/256
 * blocks of 292 B; bit-identical to the reference as compiled. */
int lg_quantize_q8_K(const float* x, int64_t n, void* y, void* stream);

/* matmul (fast/lil_math.cpp:748-776) on a pre-quantized activation:
 * out[r] = row r of w . x for r < d, n = input width.  xq holds Q8_0 blocks
 * for Q8_0/Q1_0/Q1_G weights, Q8_K blocks for Q2_K..Q6_K, and n fp32 values
 * for F32/F16 weights.  accumulate != 0 adds into out (the residual adds of
 * fast/ligguf_fast_qk.cpp:111,131). */
int lg_matvec(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, int accumulate,
              void* stream);

/* The matvec of T tokens at once on int8 MFMA (the batched prefill's GEMMs):
 * out[t*d + r] = row r of w . Q(x[t*n ..]) for t < T, r < d, each fp32 row
 * of x quantized as quantize_q8_K (K-quant weights, n % 256 == 0) or
 * quantize_q8_0 (Q8_0, Q1_0, Q1_G weights; n % 32 == 0, n % 256 for Q1_G)
 * does, or taken as fp32 (F32/F16 weights, n % 32 == 0, on fp32 MFMA).  The
 * integer block sums are those of lg_matvec (the dot products of
 * fast/lil_math.cpp:397-739); only the fp32 accumulation order differs.  Allocates and frees a workspace of
 * about 1.3*T*n bytes and synchronizes `stream` (tests and benches).  No
 * counterpart in the reference, which calls matmul per token. */
int lg_matmul_tokens(int type, const void* w, uint32_t rsz, int n, int d, const float* x, int T, float* out,
                     void* stream);

/* rmsnorm (fast/lil_math.cpp:922-929) fused with the activation quantizer
 * that follows it in inference() (:37-39): out_q gets Q8_K (qtype LG_Q8_K),
 * Q8_0 (LG_Q8_0) blocks, or with qtype LG_F32 the fp32 normalised vector.
 * out_f (optional) also receives the fp32 normalised vector. */
int lg_rmsnorm_quant(const float* x, const float* w, int n, float eps, int qtype, void* out_q, float* out_f,
                     void* stream);

/* Qwen3 per-head QK RMSNorm (fast/ligguf_fast_qk.cpp:42-51, qw/kw may be
 * NULL to skip), adjacent-pair RoPE (fast/lil_math.cpp:901-920) at `pos`,
 * and the fp16 KV write of the new row (fast/ligguf_fast_qk.cpp:57-62).
 * q [n_heads*head_dim] and k [kv_dim] are updated in place; kc_row/vc_row
 * (may be NULL) receive fp16(k), fp16(v). */
int lg_qk_norm_rope_kv(float* q, float* k, const float* v, const float* qw, const float* kw, int n_heads,
                       int n_kv_heads, int head_dim, int rope_dim, int pos, const float* freq, float eps,
                       uint16_t* kc_row, uint16_t* vc_row, void* stream);

/* GQA decode attention (fast/ligguf_fast_qk.cpp:64-105), split over the
 * sequence: out[n_heads*head_dim] = softmax(q.K^T/sqrt(hd)) V for t <= pos,
 * rows t < pos from the fp16 caches kc/vc ([pos][kv_dim] rows of this
 * layer), row pos from the fp32 k/v.  workspace must hold
 * lg_attn_workspace_size(...) bytes. */
size_t lg_attn_workspace_size(int n_heads, int head_dim, int pos);
int lg_attn_decode(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* lg_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid it).  No counterpart in the reference.  The partials go to a scratch
 * area of lg_attn_scratch_bytes() (8 MiB) that the library keeps in each
 * device's memory until the process ends; a call whose partials
 * (lg_attn_workspace_size) exceed it fails with LG_ERR_ARG -- at 32 heads of
 * 128 that is any position past 2064383.  The calling thread's current
 * device must be the one that owns the pointers and the stream.  The scratch
 * area's address on a device is looked up by lg_create on that device, else
 * by the first call there; a first call on a device under graph capture
 * fails with LG_ERR_STATE.  Nothing is allocated: every call on a device
 * shares that device's scratch area, so calls that overlap on one device
 * (other streams, other threads) race.  Same kernels and same results as
 * lg_attn_decode. */
size_t lg_attn_scratch_bytes(void);
int lg_attn_decode_noalloc(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                           int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* stream);

/* SwiGLU of fast/ligguf_fast_qk.cpp:119-123, hb[i] = silu(hb2[i]) * hb[i],
 * fused with the activation quantizer of :126 (qtype as lg_rmsnorm_quant;
 * out_q may be NULL when only hb is wanted). */
int lg_swiglu_quant(float* hb, const float* hb2, int n, int qtype, void* out_q, void* stream);

/* ===================================================================== */
/* BERT sentence embedding and the vector memory (fast/vdb.cpp)           */
/* ===================================================================== */
/* The chat driver's retrieval memory embeds every logged user turn and each
 * new user line with a BERT encoder (bert_embed, fast/vdb.cpp:123-245) and
 * searches the stored fp16 vectors by cosine similarity (vdb_query,
 * fast/vdb.cpp:337-377).  Text handling -- WordPiece tokenization
 * (bert_tokenize, :75-121), the chat-log parser (vdb_create, :269-335) and
 * the prompt text (vdb_to_prompt, :408-424) -- stays on the host; the
 * encoder and the search run here.
 *
 * Weight types: F32 and F16 matrices are used as stored and multiply fp32
 * activations (dot_f32 / dot_f16_f32, fast/lil_math.cpp:761-762); Q8_0, Q1_0
 * and Q1_G matrices multiply Q8_0-quantized activations as matmul() does for
 * them (:751-755) -- they are repacked at upload into int8 values plus one
 * fp32 scale per 32.  K-quant matrices are refused with LG_ERR_TYPE: the
 * reference's bert_embed passes no Q8_K activation for them
 * (fast/vdb.cpp:180,220,224,228). */
typedef struct lg_bert lg_bert;

/* One encoder block: bert_block (fast/lil_gguf.h:146-160).  Biases and
 * LayerNorm vectors are F32 host arrays of the matrix's output width. */
typedef struct {
    lg_weight attn_q, attn_k, attn_v, attn_out;      /* n_embed x n_embed */
    const float *attn_q_bias, *attn_k_bias, *attn_v_bias, *attn_out_bias;
    const float *attn_norm_w, *attn_norm_b;          /* attn_output_norm */
    lg_weight ffn_up;                                /* n_ff x n_embed */
    lg_weight ffn_down;                              /* n_embed x n_ff */
    const float *ffn_up_bias, *ffn_down_bias;
    const float *ffn_norm_w, *ffn_norm_b;            /* layer_output_norm */
} lg_bert_layer_desc;

/* The encoder: the BERT fields of gguf_model (fast/lil_gguf.h:200-205, read
 * by read_bert, fast/lil_gguf.cpp:501-556) and the tokenizer ids bert_embed
 * wraps a sequence with (tok_cls, tok_sep, fast/lil_gguf.cpp:384-386). */
typedef struct {
    int32_t n_layers, n_embed, n_heads, n_ff, n_context, vocab_size;
    int32_t tok_cls, tok_sep;
    float eps;                                  /* bert.attention.layer_norm_epsilon */
    lg_weight tok_embd;                         /* vocab_size x n_embed */
    lg_weight pos_embd;                         /* n_context x n_embed */
    lg_weight tok_types;                        /* >= 1 x n_embed; row 0 is used */
    const float *emb_norm_w, *emb_norm_b;       /* token_embd_norm */
    const lg_bert_layer_desc* layers;           /* n_layers entries */
} lg_bert_desc;

/* Open device `device` and create an encoder handle (no model yet).  The
 * reference keeps one static bert_runtime (fast/vdb.cpp:16-35). */
int lg_bert_create(int device, lg_bert** out);
int lg_bert_destroy(lg_bert* b);
const char* lg_bert_last_error(const lg_bert* b);

/* Copy the encoder into HBM (ensure_bert's model, fast/vdb.cpp:62-73) and
 * allocate activations for up to max_tokens tokens per pass (0: the larger
 * of n_context and 4096).  Requires n_embed % n_heads == 0, head_dim <= 128,
 * n_embed and n_ff multiples of 32. */
int lg_bert_load(lg_bert* b, const lg_bert_desc* desc, int max_tokens);

/* bert_embed (fast/vdb.cpp:123-245) after tokenization: toks are
 * bert_tokenize's ids; they are cut to n_context-2, wrapped in
 * tok_cls ... tok_sep, run through the encoder, mean-pooled over the
 * sequence and L2-normalised into out_host[n_embed].  Synchronous. */
int lg_bert_embed(lg_bert* b, const int* toks, int ntok, float* out_host);

/* Several sequences in one pass (each attends only to itself): sequence s is
 * toks[offsets[s] .. offsets[s+1]), out_host receives nseq x n_embed.  Same
 * result per sequence as lg_bert_embed; no counterpart in the reference,
 * which embeds the log's turns one at a time (fast/vdb.cpp:256,316). */
int lg_bert_embed_batch(lg_bert* b, const int* toks, const int* offsets, int nseq, float* out_host);

/* Test hook, no counterpart in the reference: the next pass (the first pass
 * of the next lg_bert_embed / _batch / lg_bert_query call) copies each Q8_0
 * activation it quantizes for a Q8_0/Q1 matrix into trace_dev, device memory
 * of lg_bert_trace_size() bytes: slot (layer l, point s) -- s = 0 the block
 * input, 1 the attention output, 2 the normalised attention-block output,
 * 3 the GELU output -- starts at (4 l + s) * lg_bert_trace_size() /
 * (4 n_layers) and holds int8 quants [T][width] followed, at max_tokens *
 * max(n_embed, n_ff) bytes, by the fp16-rounded block scales as floats
 * [width/32][T] (T: the pass's tokens, max_tokens as lg_bert_load rounded it
 * up to a multiple of 64).  Lets a test tell rounding flips of the int8
 * quantizer from arithmetic errors. */
size_t lg_bert_trace_size(const lg_bert* b);
int lg_bert_trace_next(lg_bert* b, void* trace_dev);

/* The vector memory: fp16 vectors [n][dim] in HBM (vdb_entry::vec,
 * fast/vdb.h:10-14, filled by f32_to_f16_row at fast/vdb.cpp:258).
 * lg_bert_vdb_set replaces the contents, lg_bert_vdb_append adds rows at the
 * end (vdb_create / vdb_log_turn, fast/vdb.cpp:269-335,426-436); dim must be
 * the encoder's n_embed. */
int lg_bert_vdb_set(lg_bert* b, const uint16_t* vecs_host, int n, int dim);
int lg_bert_vdb_append(lg_bert* b, const uint16_t* vecs_host, int n, int dim);
int lg_bert_vdb_size(const lg_bert* b);

/* vdb_query's search (fast/vdb.cpp:352-368) for the embedding emb_host[dim]:
 * sim_i = fp16 row i . emb; rows with sim < threshold are skipped (the
 * reference's VDB_LIKENESS_THRESHOLD is 0.75, fast/vdb.h:8); the k best
 * (k <= 8; VDB_MAX_RETRIEVAL is 3) go to idx_out/sim_out in descending
 * similarity, the lower row first among equal ones, as the reference's
 * strict-greater insertion orders them.  NaN similarities are skipped.
 * Returns the number found (0..k) or a negative LG_ERR_*. */
int lg_bert_vdb_query(lg_bert* b, const float* emb_host, int dim, float threshold, int k, int* idx_out,
                      float* sim_out);

/* vdb_query (fast/vdb.cpp:337-377) from tokens: lg_bert_embed followed by
 * the search, the embedding staying in HBM; emb_out_host (optional)
 * receives it.  Returns the number found or a negative LG_ERR_*. */
int lg_bert_query(lg_bert* b, const int* toks, int ntok, float threshold, int k, int* idx_out, float* sim_out,
                  float* emb_out_host);

#ifdef __cplusplus
}
#endif

#endif /* LIGGUF_HIP_H */
