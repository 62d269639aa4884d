/* lg_engine.hip -- context, model upload, the per-token decode step and the
 * C-ABI entry points of include/ligguf_hip.h.
 *
 * The step is the sequence of inference() (fast/ligguf_fast_qk.cpp:24-144)
 * with the math on the device:
 *   embed -> per layer { rmsnorm+quant -> QKV matvec -> QK-norm/RoPE/KV write
 *   -> split-K attention -> quant -> att_out matvec (+residual) ->
 *   rmsnorm+quant -> up|gate matvec -> SwiGLU+quant -> down matvec
 *   (+residual) } -> rmsnorm+quant -> output matvec.
 * Q|K|V and up|gate are uploaded as one matrix each when their types agree
 * (the fused row loops of matmul3/matmul2, fast/lil_math.cpp:779-899).
 *
 * Device layout (HBM): weights as stored in GGUF rows; the fp16 KV cache
 * [n_layers][n_context][kv_dim] as model_state (fast/common.cpp:31-32);
 * fp32 activations x, q|k|v, att, hb|hb2, logits; quantized activations
 * in Q8_K and/or Q8_0 form.
 */
#include <algorithm>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include <string>
#include <initializer_list>
#include <vector>

#include "lg_common.h"
#include "lg_persist.h"
#include "lg_prefill.h"

/* ------------------------------------------------------------------ */
/* errors                                                               */
/* ------------------------------------------------------------------ */
static thread_local char g_err[1024];

void lg_set_error(const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char* lg_get_thread_error(void) { return g_err; }

int lg_check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        lg_set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return LG_ERR_HIP;
    }
    return LG_OK;
}

extern "C" int64_t lg_row_size(int type, int64_t n)
{
    if (n < 0) return -1;
    switch (type) {
    case LG_F32: return 4 * n;
    case LG_F16: return 2 * n;
    case LG_Q8_0: return n % 32 ? -1 : n / 32 * LG_BS_Q8_0;
    case LG_Q1_0: return n % 32 ? -1 : n / 32 * LG_BS_Q1_0;
    case LG_Q1_G: return n % 128 ? -1 : n / 128 * LG_BS_Q1_G;
    case LG_Q2_K: return n % 256 ? -1 : n / 256 * LG_BS_Q2_K;
    case LG_Q3_K: return n % 256 ? -1 : n / 256 * LG_BS_Q3_K;
    case LG_Q4_K: return n % 256 ? -1 : n / 256 * LG_BS_Q4_K;
    case LG_Q5_K: return n % 256 ? -1 : n / 256 * LG_BS_Q5_K;
    case LG_Q6_K: return n % 256 ? -1 : n / 256 * LG_BS_Q6_K;
    case LG_Q8_K: return n % 256 ? -1 : n / 256 * LG_BS_Q8_K;
    default: return -1;
    }
}

/* activation family a weight type consumes */
enum { ACT_K = 1, ACT_80 = 2, ACT_F = 4 };
static int act_family(int type)
{
    switch (type) {
    case LG_Q2_K: case LG_Q3_K: case LG_Q4_K: case LG_Q5_K: case LG_Q6_K: return ACT_K;
    case LG_Q8_0: case LG_Q1_0: case LG_Q1_G: return ACT_80;
    case LG_F32: case LG_F16: return ACT_F;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ */
/* context                                                              */
/* ------------------------------------------------------------------ */
struct dweight {
    uint8_t* data = nullptr;
    int type = -1;
    uint32_t rsz = 0;
    int rows = 0, cols = 0;
};

struct dlayer {
    float *att_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    dweight q, k, v;        /* views into qkv when fused */
    bool qkv_fused = false;
    bool qk_fused = false;  /* Q|K stacked in qkv, V of another type on its own */
    dweight qkv;
    dweight att_out;
    dweight up, gate;
    bool ug_fused = false;
    dweight ug;
    dweight down;
};

struct lg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    char err[1024] = {0};
    std::vector<void*> allocs;

    bool loaded = false;
    int arch = 0, n_layers = 0, n_embed = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, kv_dim = 0, n_ff = 0;
    int vocab = 0, n_context = 0, rope_dim = 0;
    float eps = 0.0f;
    std::vector<dlayer> layers;
    dweight embd, output;
    float* out_norm = nullptr;
    float* rope_freq = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;

    float *x = nullptr, *qkv = nullptr, *att = nullptr, *hb = nullptr, *logits = nullptr, *xf = nullptr;
    uint8_t *xqk = nullptr, *xq0 = nullptr;
    float* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    int* argmax_dev = nullptr;
    LgSampleWs* samp = nullptr;  /* top-p sampler workspace, vocab entries */

    /* persistent one-launch-per-token path (lg_persist.hip) */
    bool pk_ok = false;          /* the loaded model fits it */
    int path = LG_PATH_AUTO;
    int pk_nwg = 0;
    size_t pk_cnt_bytes = 0;     /* the zeroed block of counters and flags */
    PkParams pk = {};
    const void* pk_kernel = nullptr; /* the instantiation for this model */
    uint64_t* pk_trace = nullptr;    /* phase timestamps of the next persistent step */
    uint8_t* act_trace = nullptr;    /* quantized activations of the next step (any path) */
    size_t act_stride = 0;           /* bytes per activation slot of that trace */
    uint64_t pk_base = 0;
    int* pk_status_host = nullptr;   /* pinned {token, error} of the last persistent / fused step */
    bool last_was_pk = false;        /* the last step left its greedy token in pk_status_host */

    /* fused per-phase kernels replayed from a HIP graph (lg_fused.hip) */
    const void* fused_fn = nullptr;
    std::vector<PkLayer> pk_layers;  /* host copy: the fused kernels take their layer by value */
    /* layer matrices and norms of models with one shape and type per matrix
     * kind: one allocation per kind, layer l at l * stride */
    struct {
        bool ok;
        uint8_t *qkv, *ao, *ug, *down;
        size_t qkv_b, ao_b, ug_b, down_b;
        float *att_norm, *ffn_norm, *q_norm, *k_norm;
    } arena = {};
    /* batched prefill */
    bool pf_ok = false;
    int pf_fam = 0;                  /* activation forms of the model's matrices: bit 0 Q8_K, bit 1 Q8_0 */
    uint8_t* pf_trace = nullptr;     /* quantized activations of every token of the next batched prefill */
    int prefill_path = LG_PREFILL_AUTO;
    std::vector<PfLayer> pf_layers;
    PfModel pf_model = {};
    PfBuffers pf = {};
    PkStep* step_dev = nullptr;      /* {tok, pos, feed_end} the next fused step reads */
    PkStep* step_ring = nullptr;     /* pinned slots for host updates of step_dev */
    int ring_next = 0, ring_pending = 0;
    int* feed_dev = nullptr;         /* [n_context] prompt tokens */
    int* feed_host = nullptr;        /* pinned staging of the same */
    bool dev_known = false;          /* step_dev holds {dev_tok, dev_pos} (read back after a sync) */
    int dev_tok = 0, dev_pos = 0, dev_feed_end = 0, last_pos = 0;
    bool use_graph = true;
    bool regroup = true;             /* fused kernels read regrouped copies of misaligned formats */
    bool qkva = true;                /* fused step: QKV and short-context attention in one kernel */
    bool qkvao = true;               /* ... and att_out, split by KV group */
    hipGraphExec_t graph[2] = {nullptr, nullptr};   /* the step with short / long-context attention */
};

static int ctx_fail(lg_ctx* ctx, int rc)
{
    if (ctx && rc != LG_OK) snprintf(ctx->err, sizeof(ctx->err), "%s", g_err);
    return rc;
}

static int dalloc(lg_ctx* ctx, void** p, size_t bytes)
{
    const hipError_t e = hipMalloc(p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        lg_set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        return LG_ERR_NOMEM;
    }
    ctx->allocs.push_back(*p);
    return LG_OK;
}

static void free_model(lg_ctx* ctx)
{
    for (void* p : ctx->allocs) hipFree(p);
    ctx->allocs.clear();
    ctx->layers.clear();
    ctx->loaded = false;
    ctx->pk_ok = false;
    ctx->last_was_pk = false;
    ctx->pk_base = 0;
    ctx->fused_fn = nullptr;
    ctx->dev_known = false;
    ctx->dev_feed_end = 0;
    ctx->pf_ok = false;
    ctx->pf_fam = 0;
    ctx->pf_trace = nullptr;
    ctx->arena = {};
    ctx->pf_layers.clear();
    ctx->pf = PfBuffers{};
    for (auto& gr : ctx->graph) {
        if (gr) hipGraphExecDestroy(gr);
        gr = nullptr;
    }
}

extern "C" int lg_create(int device, lg_ctx** out)
{
    if (!out) { lg_set_error("lg_create: null output"); return LG_ERR_ARG; }
    lg_rand_guard keep_rand;
    *out = nullptr;
    int n = 0;
    LG_HIP_CHECK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) { lg_set_error("lg_create: device %d of %d", device, n); return LG_ERR_ARG; }
    LG_HIP_CHECK(hipSetDevice(device));
    int rc = lg_attn_scratch_setup();   /* before any caller's graph capture on this device */
    if (rc) return rc;
    lg_ctx* ctx = new lg_ctx();
    ctx->device = device;
    const char* ng = getenv("LG_NO_GRAPH");
    ctx->use_graph = !(ng && ng[0] == '1');
    const char* nr = getenv("LG_NO_REGROUP");
    ctx->regroup = !(nr && nr[0] == '1');
    const char* nq = getenv("LG_NO_QKVA");
    ctx->qkva = !(nq && nq[0] == '1');
    const char* no = getenv("LG_NO_QKVAO");
    ctx->qkvao = !(no && no[0] == '1');
    const hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        lg_set_error("hipStreamCreate failed: %s", hipGetErrorString(e));
        delete ctx;
        return LG_ERR_HIP;
    }
    *out = ctx;
    return LG_OK;
}

extern "C" int lg_destroy(lg_ctx* ctx)
{
    if (!ctx) return LG_OK;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    free_model(ctx);
    lg_sample_ws_free(ctx->samp);
    if (ctx->pk_status_host) hipHostFree(ctx->pk_status_host);
    if (ctx->step_ring) hipHostFree(ctx->step_ring);
    if (ctx->feed_host) hipHostFree(ctx->feed_host);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return LG_OK;
}

extern "C" const char* lg_last_error(const lg_ctx* ctx) { return ctx ? ctx->err : g_err; }

/* ------------------------------------------------------------------ */
/* model upload                                                         */
/* ------------------------------------------------------------------ */
static int check_weight(const lg_weight& w, int rows, int cols, const char* name)
{
    if (!w.data) { lg_set_error("load_model: %s missing", name); return LG_ERR_ARG; }
    if (w.rows != rows || w.cols != cols) {
        lg_set_error("load_model: %s is %dx%d, expected %dx%d", name, w.rows, w.cols, rows, cols);
        return LG_ERR_ARG;
    }
    if (!act_family(w.type)) { lg_set_error("load_model: %s has unsupported type %d", name, w.type); return LG_ERR_TYPE; }
    const int64_t need = lg_row_size(w.type, cols);
    if (need < 0 || (int64_t)w.rsz < need) { lg_set_error("load_model: %s row size %u (type %d needs %lld)", name, w.rsz, w.type, (long long)need); return LG_ERR_ARG; }
    return LG_OK;
}

/* Host-to-device copies of the model through two pinned staging buffers: the
 * CPU copies the next chunk from the caller's (pageable, often mmap-ed) tensor
 * into one buffer while the DMA engine moves the other, so the upload runs
 * at the pinned transfer rate instead of a pageable copy's. */
struct lg_uploader {
    static constexpr size_t CHUNK = (size_t)32 << 20;
    uint8_t* pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int cur = 0;
    hipStream_t s = nullptr;
    size_t bytes = 0;

    int init(hipStream_t stream)
    {
        s = stream;
        for (int i = 0; i < 2; i++) {
            LG_HIP_CHECK(hipHostMalloc((void**)&pin[i], CHUNK, 0));
            LG_HIP_CHECK(hipEventCreateWithFlags(&done[i], hipEventDisableTiming));
        }
        return LG_OK;
    }
    int copy(void* dst, const void* src, size_t n)
    {
        const uint8_t* h = (const uint8_t*)src;
        uint8_t* d = (uint8_t*)dst;
        while (n) {
            const size_t c = n < CHUNK ? n : CHUNK;
            if (used[cur]) LG_HIP_CHECK(hipEventSynchronize(done[cur]));   /* its last DMA has finished */
            memcpy(pin[cur], h, c);
            LG_HIP_CHECK(hipMemcpyAsync(d, pin[cur], c, hipMemcpyHostToDevice, s));
            LG_HIP_CHECK(hipEventRecord(done[cur], s));
            used[cur] = true;
            cur ^= 1;
            h += c; d += c; n -= c;
            bytes += c;
        }
        return LG_OK;
    }
    int finish() { LG_HIP_CHECK(hipStreamSynchronize(s)); return LG_OK; }
    ~lg_uploader()
    {
        if (s) hipStreamSynchronize(s);
        for (int i = 0; i < 2; i++) {
            if (pin[i]) hipHostFree(pin[i]);
            if (done[i]) hipEventDestroy(done[i]);
        }
    }
};
static thread_local lg_uploader* g_up = nullptr;   /* set for the duration of one lg_load_model */

static int h2d(void* dst, const void* src, size_t n)
{
    if (g_up) return g_up->copy(dst, src, n);
    LG_HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    return LG_OK;
}

static int upload_weight(lg_ctx* ctx, const lg_weight& w, dweight& d, uint8_t* dst = nullptr)
{
    const size_t bytes = (size_t)w.rows * w.rsz;
    int rc = dst ? (d.data = dst, LG_OK) : dalloc(ctx, (void**)&d.data, bytes);
    if (rc) return rc;
    if ((rc = h2d(d.data, w.data, bytes))) return rc;
    d.type = w.type; d.rsz = w.rsz; d.rows = w.rows; d.cols = w.cols;
    return LG_OK;
}

/* stack matrices of one type and row size into one device matrix */
static int upload_stacked(lg_ctx* ctx, const lg_weight* const* ws, int n, dweight& out, dweight* views,
                          uint8_t* dst = nullptr)
{
    size_t bytes = 0;
    int rows = 0;
    for (int i = 0; i < n; i++) { bytes += (size_t)ws[i]->rows * ws[i]->rsz; rows += ws[i]->rows; }
    int rc = dst ? (out.data = dst, LG_OK) : dalloc(ctx, (void**)&out.data, bytes);
    if (rc) return rc;
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        const size_t b = (size_t)ws[i]->rows * ws[i]->rsz;
        if ((rc = h2d(out.data + off, ws[i]->data, b))) return rc;
        views[i].data = out.data + off;
        views[i].type = ws[i]->type; views[i].rsz = ws[i]->rsz; views[i].rows = ws[i]->rows; views[i].cols = ws[i]->cols;
        off += b;
    }
    out.type = ws[0]->type; out.rsz = ws[0]->rsz; out.rows = rows; out.cols = ws[0]->cols;
    return LG_OK;
}

static int upload_floats(lg_ctx* ctx, const float* h, size_t n, float** d, const char* name, float* dst = nullptr)
{
    if (!h) { lg_set_error("load_model: %s missing", name); return LG_ERR_ARG; }
    int rc = dst ? (*d = dst, LG_OK) : dalloc(ctx, (void**)d, n * sizeof(float));
    if (rc) return rc;
    return h2d(*d, h, n * sizeof(float));
}

/* ------------------------------------------------------------------ */
/* persistent path set-up                                               */
/* ------------------------------------------------------------------ */
#define LG_STEP_RING 64   /* pinned step records in flight before a forced sync */
/* the persistent kernel reads every layer matrix at width n_embed = 4096
 * (n_ff = 12288 for down), one type for all layer matrices */
/* Rows regrouped for the fused kernels' aligned loads (Fmt<LG_Q8_0_R>,
 * Fmt<LG_Q6_K_R>, Fmt<LG_Q1_G_R>): each run of 8 blocks of a row becomes its
 * quants, then its scales (Q6_K: ql, qh, scales, d).  Only for widths of
 * whole groups on 16-byte row boundaries; empty otherwise. */
static std::vector<uint8_t> repack_rows(const lg_weight& w)
{
    std::vector<uint8_t> out;
    if (!w.data || w.cols <= 0) return out;
    const bool q8 = w.type == LG_Q8_0 && w.cols % 256 == 0;
    const bool q6 = w.type == LG_Q6_K && w.cols % 2048 == 0;
    const bool q1 = w.type == LG_Q1_G && w.cols % 1024 == 0;
    const bool q3 = w.type == LG_Q3_K && w.cols % 2048 == 0;
    const bool q0 = w.type == LG_Q1_0 && w.cols % 256 == 0;
    if (!q8 && !q6 && !q1 && !q3 && !q0) return out;
    const size_t bs = q8 ? LG_BS_Q8_0 : q6 ? LG_BS_Q6_K : q1 ? LG_BS_Q1_G : q0 ? LG_BS_Q1_0 : LG_BS_Q3_K;
    const size_t ng = (size_t)w.cols / ((q8 || q0) ? 256 : q1 ? 1024 : 2048);
    if (w.rsz != ng * 8 * bs) return out;
    out.resize((size_t)w.rows * w.rsz);
    const uint8_t* src = (const uint8_t*)w.data;
    for (size_t r = 0; r < (size_t)w.rows; r++)
        for (size_t g = 0; g < ng; g++) {
            const uint8_t* in = src + r * w.rsz + g * 8 * bs;
            uint8_t* o = out.data() + r * w.rsz + g * 8 * bs;
            for (int j = 0; j < 8; j++) {
                const uint8_t* b = in + j * bs;
                if (q8) {
                    memcpy(o + 256 + 2 * j, b, 2);          /* d */
                    memcpy(o + 32 * j, b + 2, 32);          /* qs */
                } else if (q0) {
                    memcpy(o + 32 + 2 * j, b, 2);           /* d */
                    memcpy(o + 4 * j, b + 2, 4);            /* sign bits */
                } else if (q1) {
                    memcpy(o + 128 + 2 * j, b, 2);          /* d */
                    memcpy(o + 16 * j, b + 2, 16);          /* sign bits */
                } else if (q3) {
                    memcpy(o + 32 * j, b, 32);              /* hmask */
                    memcpy(o + 256 + 64 * j, b + 32, 64);   /* qs */
                    memcpy(o + 768 + 12 * j, b + 96, 12);   /* scales */
                    memcpy(o + 864 + 2 * j, b + 108, 2);    /* d */
                } else {
                    memcpy(o + 128 * j, b, 128);            /* ql */
                    memcpy(o + 1024 + 64 * j, b + 128, 64); /* qh */
                    memcpy(o + 1536 + 16 * j, b + 192, 16); /* scales */
                    memcpy(o + 1664 + 2 * j, b + 208, 2);   /* d */
                }
            }
        }
    return out;
}

static bool pk_shape_ok(const dweight& w, int type, int rows, int cols)
{
    return w.type == type && w.rows == rows && w.cols == cols;
}

static int setup_persistent(lg_ctx* ctx, const lg_model_desc* m)
{
    ctx->pk_ok = false;
    ctx->pk_kernel = nullptr;
    const int nrep = m->n_heads / m->n_kv_heads;
    const int lt = ctx->layers.empty() ? -1 : ctx->layers[0].q.type;
    /* attention partials per head and layer: PK_ATT_MERGE chunks, or the
     * long-context chunk count of pk_attn_split (one grid of one workgroup
     * per CU) at the longest context */
    int dev = 0, ncu = 0;
    LG_HIP_CHECK(hipGetDevice(&dev));
    LG_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    int att_chunk = 0, att_nch = 0;
    const int att_max = m->n_kv_heads > 0 ? ncu * LG_ATT_WGS / m->n_kv_heads : 0;
    if (m->head_dim > 0 && m->head_dim <= 128 && nrep >= 1 && nrep <= PK_MAX_NREP && m->n_kv_heads > 0)
        pk_attn_split(m->n_context, m->head_dim, nrep, att_max, &att_chunk, &att_nch);
    /* slots for the most chunks any position takes: the chunk size is
     * rounded up to whole steps, so a shorter context can take more chunks
     * than n_context does (up to the clamped att_max, never more) */
    att_nch = std::max(std::min(std::max(att_max, PK_ATT_MERGE), PK_ATT_MAX_NCH), PK_ATT_MERGE);
    /* widths: any the activation builds hold (LDS staging of n_embed and of
     * the quantized n_ff vector -- the fp32 one for F16 / F32 layers), in whole
     * 256-value Q8_K blocks for K-quant and Q1_G layers; which widths have
     * kernels is up to the variants */
    const bool fact = lt == LG_F16 || lt == LG_F32;
    const bool q8act = lt == LG_Q8_0 || lt == LG_Q1_0 || fact;
    bool ok = m->n_embed <= PK_MAX_EMBED && m->n_ff <= (fact ? PK_MAX_FF_F : PK_MAX_FF) &&
              m->n_embed % (q8act ? 32 : 256) == 0 &&
              m->n_ff % (q8act ? 32 : 256) == 0 && att_chunk > 0 && att_nch <= PK_ATT_MAX_NCH &&
              m->n_kv_heads <= 32 && m->n_heads <= 64 && ctx->output.cols == m->n_embed;
    /* uniform: every layer matrix of type lt (the persistent kernel's and
     * the fused step's case); otherwise the fused step also takes layers
     * whose V (Q|K stacked) and down matrices are of a side type */
    bool uniform = ok && ctx->arena.ok;
    for (int l = 0; ok && l < m->n_layers; l++) {
        const dlayer& D = ctx->layers[l];
        const int ne = m->n_embed, kvd = m->kv_dim;
        const bool qkv_u = D.qkv_fused && pk_shape_ok(D.qkv, lt, ne + 2 * kvd, ne);
        const bool qkv_m = D.qk_fused && pk_shape_ok(D.qkv, lt, ne + kvd, ne) && lg_fused_side_type(lt, D.v.type) &&
                           pk_shape_ok(D.v, D.v.type, kvd, ne);
        const bool down_u = pk_shape_ok(D.down, lt, ne, m->n_ff);
        const bool down_m = lg_fused_side_type(lt, D.down.type) && pk_shape_ok(D.down, D.down.type, ne, m->n_ff);
        ok = D.ug_fused && pk_shape_ok(D.att_out, lt, ne, ne) && pk_shape_ok(D.ug, lt, 2 * m->n_ff, ne) &&
             (qkv_u || qkv_m) && (down_u || down_m);
        uniform = uniform && qkv_u && down_u;
    }
    uniform = uniform && ok;
    /* the fused kernels come in width classes; the persistent kernel is
     * instantiated for n_embed 4096 / n_ff 12288 only */
    const void* fused = ok ? lg_fused_variant(lt, ctx->output.type, m->head_dim, nrep, m->n_embed, m->n_ff) : nullptr;
    const void* kern = uniform && m->n_embed == 4096 && m->n_ff == 3 * m->n_embed
                           ? lg_persist_kernel(lt, ctx->output.type, m->head_dim, nrep)
                           : nullptr;
    if (!kern && !fused) return LG_OK;   /* the multi-kernel path serves this model */
    int rc;
    if (kern) {
        if ((rc = lg_persist_grid(kern, &ctx->pk_nwg))) return rc;
    } else {
        ctx->pk_nwg = ncu;   /* one workgroup per CU, as the persistent grid */
    }
    std::vector<PkLayer> hl(m->n_layers);
    /* uniform Q8_0 / Q6_K / Q1_G layers: the fused kernels read regrouped
     * copies of every layer matrix (aligned loads); the persistent kernel
     * keeps the GGUF rows of the arenas -- same values, same results */
    const int gw = (lt == LG_Q8_0 || lt == LG_Q1_0) ? 256 : (lt == LG_Q6_K || lt == LG_Q3_K) ? 2048
                 : lt == LG_Q1_G ? 1024 : 0;
#ifndef LG_REP_LAYERS
#define LG_REP_LAYERS 1
#endif
    const bool rep_layers = LG_REP_LAYERS && ctx->regroup && fused && uniform && gw && m->n_embed % gw == 0 &&
                            m->n_ff % gw == 0;
    auto upload_rep = [&](std::initializer_list<const lg_weight*> ws, const uint8_t*& ptr) -> int {
        std::vector<uint8_t> all;
        for (const lg_weight* w : ws) {
            const std::vector<uint8_t> rp = repack_rows(*w);
            if (rp.empty()) { lg_set_error("load_model: regrouping a layer matrix failed"); return LG_ERR_ARG; }
            all.insert(all.end(), rp.begin(), rp.end());
        }
        uint8_t* d = nullptr;
        int rc2;
        if ((rc2 = dalloc(ctx, (void**)&d, all.size()))) return rc2;
        if ((rc2 = h2d(d, all.data(), all.size()))) return rc2;
        ptr = d;
        return LG_OK;
    };
    for (int l = 0; l < m->n_layers; l++) {
        const dlayer& D = ctx->layers[l];
        PkLayer& P = hl[l];
        P.qkv = D.qkv.data; P.qkv_rsz = D.qkv.rsz; P.qkv_t = D.qkv.type;
        P.ao = D.att_out.data; P.ao_rsz = D.att_out.rsz; P.ao_t = D.att_out.type;
        P.ug = D.ug.data; P.ug_rsz = D.ug.rsz; P.ug_t = D.ug.type;
        P.down = D.down.data; P.down_rsz = D.down.rsz; P.down_t = D.down.type;
        P.v = D.qk_fused ? D.v.data : nullptr; P.v_rsz = D.v.rsz; P.v_t = D.v.type;
        if (!kern && ctx->regroup) {
            /* a mixed layer's Q6_K V and down matrices: the fused kernels read
             * regrouped copies (aligned loads, Fmt<LG_Q6_K_R>) */
            const lg_layer_desc& ML = m->layers[l];
            auto regroup = [&](const lg_weight& w, const uint8_t*& ptr, int& t) -> int {
                if (w.type != LG_Q6_K || w.type == lt) return LG_OK;
                const std::vector<uint8_t> rp = repack_rows(w);
                if (rp.empty()) return LG_OK;
                uint8_t* d = nullptr;
                int rc2;
                if ((rc2 = dalloc(ctx, (void**)&d, rp.size()))) return rc2;
                if ((rc2 = h2d(d, rp.data(), rp.size()))) return rc2;
                ptr = d;
                t = LG_Q6_K_R;
                return LG_OK;
            };
            if (P.v && (rc = regroup(ML.att_v, P.v, P.v_t))) return rc;
            if ((rc = regroup(ML.ffn_down, P.down, P.down_t))) return rc;
        }
        if (rep_layers) {
            const lg_layer_desc& ML = m->layers[l];
            const int rt = lt == LG_Q8_0 ? LG_Q8_0_R : lt == LG_Q6_K ? LG_Q6_K_R : lt == LG_Q3_K ? LG_Q3_K_R
                         : lt == LG_Q1_0 ? LG_Q1_0_R : LG_Q1_G_R;
            if ((rc = upload_rep({&ML.att_q, &ML.att_k, &ML.att_v}, P.qkv))) return rc;
            if ((rc = upload_rep({&ML.att_out}, P.ao))) return rc;
            if ((rc = upload_rep({&ML.ffn_up, &ML.ffn_gate}, P.ug))) return rc;
            if ((rc = upload_rep({&ML.ffn_down}, P.down))) return rc;
            P.qkv_t = P.ao_t = P.ug_t = P.down_t = rt;
        }
        P.att_norm = D.att_norm; P.ffn_norm = D.ffn_norm; P.q_norm = D.q_norm; P.k_norm = D.k_norm;
    }
    PkLayer* dl = nullptr;
    if ((rc = dalloc(ctx, (void**)&dl, hl.size() * sizeof(PkLayer)))) return rc;
    LG_HIP_CHECK(hipMemcpy(dl, hl.data(), hl.size() * sizeof(PkLayer), hipMemcpyHostToDevice));
    ctx->pk_layers = hl;
    PkParams& P = ctx->pk;
    P = PkParams{};
    P.layers = dl;
    P.w_qkv = ctx->arena.qkv; P.w_ao = ctx->arena.ao; P.w_ug = ctx->arena.ug; P.w_down = ctx->arena.down;
    P.s_qkv = ctx->arena.qkv_b; P.s_ao = ctx->arena.ao_b; P.s_ug = ctx->arena.ug_b; P.s_down = ctx->arena.down_b;
    P.n_att = ctx->arena.att_norm; P.n_ffn = ctx->arena.ffn_norm; P.n_q = ctx->arena.q_norm; P.n_k = ctx->arena.k_norm;
    P.n_layers = m->n_layers; P.n_embed = m->n_embed; P.n_heads = m->n_heads; P.n_kv = m->n_kv_heads;
    P.head_dim = m->head_dim; P.kv_dim = m->kv_dim; P.n_ff = m->n_ff; P.vocab = m->vocab_size;
    P.n_ctx = m->n_context; P.rope_dim = m->rope_dim; P.eps = m->rms_epsilon;
    P.embd = ctx->embd.data; P.embd_rsz = ctx->embd.rsz; P.embd_t = ctx->embd.type;
    P.out_w = ctx->output.data; P.out_rsz = ctx->output.rsz; P.out_t = ctx->output.type;
    P.out_wr = nullptr;
    P.layers_rep = rep_layers ? 1 : 0;
    if (fused && ctx->regroup) {
        const std::vector<uint8_t> rp = repack_rows(m->output);
        if (!rp.empty()) {
            uint8_t* d = nullptr;
            if ((rc = dalloc(ctx, (void**)&d, rp.size()))) return rc;
            if ((rc = h2d(d, rp.data(), rp.size()))) return rc;
            P.out_wr = d;
        }
    }
    P.out_norm = ctx->out_norm; P.rope_freq = ctx->rope_freq;
    P.kc = ctx->kc; P.vc = ctx->vc;
    P.logits = ctx->logits;
    {
        /* per-layer activation buffers, each written once per step */
        const size_t L = (size_t)m->n_layers, ne = m->n_embed, qs = ne + 2 * m->kv_dim, ff = m->n_ff;
        const size_t floats = (L + 1) * ne + L * ne + L * qs + L * ff;
        float* arena = nullptr;
        if ((rc = dalloc(ctx, (void**)&arena, floats * sizeof(float)))) return rc;
        P.xs = arena;
        P.xm = P.xs + (L + 1) * ne;
        P.qkv = P.xm + L * ne;
        P.hb = P.qkv + L * qs;
    }
    {
        /* per-layer attention partials, each written once per step */
        const size_t L = (size_t)m->n_layers;
        float* ws = nullptr;
        /* chunks (at least the short path's), then the merged groups */
        const size_t slots = (size_t)std::max(att_nch, PK_ATT_MERGE) + PK_ATT_MERGE;
        if ((rc = dalloc(ctx, (void**)&ws, L * slots * ((size_t)m->n_embed + 2 * m->n_heads) * sizeof(float))))
            return rc;
        P.att_slots = (int)slots;
        P.att_grid = ncu * LG_ATT_WGS;
        P.att_po = ws;
        P.att_pml = ws + L * slots * m->n_embed;
    }
    /* att_out partials of the 8 KV groups (one layer at a time: the next
     * layer's kernel writes them after this layer's up|gate read them) */
    if ((rc = dalloc(ctx, (void**)&P.ao_part, 8 * (size_t)m->n_embed * sizeof(float)))) return rc;
    /* one zeroed block for the counters and flags; argmax partials for up
     * to LG_OUT_MAX_WGS output-head workgroups per CU */
    const int nwg = ctx->pk_nwg;
    const size_t namax = (size_t)nwg * LG_OUT_MAX_WGS;
    const size_t cnt_bytes = (size_t)nwg * 8 + namax * 8 + 256 + 32 * PK_ATT_MERGE * 4 + LG_MAX_GROUP_WORDS * 8;
    uint8_t* blk = nullptr;
    if ((rc = dalloc(ctx, (void**)&blk, cnt_bytes))) return rc;
    LG_HIP_CHECK(hipMemset(blk, 0, cnt_bytes));
    ctx->pk_cnt_bytes = cnt_bytes;
    P.progress = (uint64_t*)blk;                                   /* nwg x 8 B */
    P.amax_v = (float*)(blk + (size_t)nwg * 8);                    /* namax x 4 B */
    P.amax_i = (int*)(blk + (size_t)nwg * 8 + namax * 4);          /* namax x 4 B */
    uint8_t* tail = blk + (size_t)nwg * 8 + namax * 8;
    P.amax_cnt = (uint32_t*)tail;
    P.tok_out = (int*)(tail + 64);                                 /* {token, error} */
    P.err = (uint32_t*)(tail + 68);
    P.attn_cnt = (uint32_t*)(tail + 256);                          /* up to 32 heads x PK_ATT_MERGE groups */
    P.grp_cnt = (uint64_t*)(tail + 256 + 32 * PK_ATT_MERGE * 4);   /* LG_MAX_GROUP_WORDS x 8 B */
    P.qkva = ctx->qkva;
    P.qkvao = ctx->qkvao;
    P.spin_cap = 1 << 20;
    P.act_stride = ctx->act_stride;
    /* fused path: device step record, prompt feed, pinned staging */
    if ((rc = dalloc(ctx, (void**)&ctx->step_dev, sizeof(PkStep)))) return rc;
    LG_HIP_CHECK(hipMemset(ctx->step_dev, 0, sizeof(PkStep)));
    if ((rc = dalloc(ctx, (void**)&P.tok_hist, (size_t)m->n_context * sizeof(int)))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->feed_dev, (size_t)m->n_context * sizeof(int)))) return rc;
    LG_HIP_CHECK(hipMemset(ctx->feed_dev, 0, (size_t)m->n_context * sizeof(int)));
    P.feed = ctx->feed_dev;
    if (ctx->feed_host) { hipHostFree(ctx->feed_host); ctx->feed_host = nullptr; }
    LG_HIP_CHECK(hipHostMalloc((void**)&ctx->feed_host, (size_t)m->n_context * sizeof(int), 0));
    if (!ctx->step_ring) LG_HIP_CHECK(hipHostMalloc((void**)&ctx->step_ring, LG_STEP_RING * sizeof(PkStep), 0));
    ctx->ring_next = ctx->ring_pending = 0;
    ctx->fused_fn = fused;
    if (!ctx->pk_status_host) LG_HIP_CHECK(hipHostMalloc((void**)&ctx->pk_status_host, 2 * sizeof(int), 0));
    ctx->pk_base = 0;
    ctx->pk_kernel = kern;
    ctx->pk_ok = true;
    return LG_OK;
}

/* the persistent kernel's counters after an expired wait: back to zero */
static void pk_reset(lg_ctx* c)
{
    hipMemsetAsync(c->pk.progress, 0, c->pk_cnt_bytes, c->stream);
    hipStreamSynchronize(c->stream);
    c->pk_base = 0;
}

/* AUTO takes the multi-kernel path until the persistent kernel measures
 * faster on the headline workload; PERSISTENT selects it explicitly */
static bool use_pk(const lg_ctx* c) { return c->pk_ok && c->pk_kernel && c->path == LG_PATH_PERSISTENT; }
static bool use_fused(const lg_ctx* c)
{
    return c->pk_ok && c->fused_fn && (c->path == LG_PATH_FUSED || c->path == LG_PATH_AUTO);
}

/* write {tok, pos, feed_end} into the device step record through a pinned slot */
static int fused_set_step(lg_ctx* c, int tok, int pos, int feed_end, uint64_t* trace = nullptr)
{
    if (c->ring_pending >= LG_STEP_RING) {
        LG_HIP_CHECK(hipStreamSynchronize(c->stream));
        c->ring_pending = 0;
    }
    PkStep* s = &c->step_ring[c->ring_next];
    c->ring_next = (c->ring_next + 1) % LG_STEP_RING;
    c->ring_pending++;
    memset(s, 0, sizeof(*s));
    s->tok = tok; s->pos = pos; s->feed_end = feed_end; s->trace = trace;
    LG_HIP_CHECK(hipMemcpyAsync(c->step_dev, s, sizeof(PkStep), hipMemcpyHostToDevice, c->stream));
    c->dev_feed_end = feed_end;
    return LG_OK;
}

/* attention at position pos takes the long-context kernel */
static bool att_long(const lg_ctx* c, int pos)
{
    return pk_att_long(pos, c->pk.head_dim, c->pk.n_heads / c->pk.n_kv, c->pk.n_kv, c->pk_nwg);
}

/* one fused step at position pos on the stream: its graph (captured on first
 * use; one per attention kernel) or the same launches issued directly (a
 * step with an activation trace is always launched directly) */
static int fused_launch(lg_ctx* c, int pos, uint8_t* act_trace = nullptr)
{
    const bool lc = att_long(c, pos);
    if (act_trace)
        return lg_fused_enqueue(c->fused_fn, c->pk, c->pk_layers.data(), c->step_dev, c->n_layers, c->pk_nwg, lc,
                                c->stream, act_trace);
    hipGraphExec_t& graph = c->graph[lc ? 1 : 0];
    if (c->use_graph && !graph) {
        hipGraph_t g = nullptr;
        LG_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        const int rc = lg_fused_enqueue(c->fused_fn, c->pk, c->pk_layers.data(), c->step_dev, c->n_layers, c->pk_nwg,
                                        lc, c->stream);
        const hipError_t ec = hipStreamEndCapture(c->stream, &g);
        if (rc || ec != hipSuccess) {
            if (g) hipGraphDestroy(g);
            lg_set_error("graph capture of the fused step failed: %s", hipGetErrorString(ec));
            return rc ? rc : LG_ERR_HIP;
        }
        const hipError_t ei = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (ei != hipSuccess) {
            graph = nullptr;
            lg_set_error("graph instantiate: %s", hipGetErrorString(ei));
            return LG_ERR_HIP;
        }
    }
    if (c->use_graph) {
        LG_HIP_CHECK(hipGraphLaunch(graph, c->stream));
        return LG_OK;
    }
    return lg_fused_enqueue(c->fused_fn, c->pk, c->pk_layers.data(), c->step_dev, c->n_layers, c->pk_nwg, lc, c->stream);
}

static int enqueue_fused(lg_ctx* c, int tok, int pos)
{
    int rc;
    if (c->pk_trace || !(c->dev_known && c->dev_tok == tok && c->dev_pos == pos && pos >= c->dev_feed_end))
        if ((rc = fused_set_step(c, tok, pos, 0, c->pk_trace))) return rc;
    uint8_t* atr = c->act_trace;
    c->pk_trace = nullptr;
    c->act_trace = nullptr;
    c->dev_known = false;
    if ((rc = fused_launch(c, pos, atr))) return rc;
    LG_HIP_CHECK(hipMemcpyAsync(c->pk_status_host, c->pk.tok_out, 2 * sizeof(int), hipMemcpyDeviceToHost, c->stream));
    c->last_was_pk = true;
    c->last_pos = pos;
    return LG_OK;
}

static int enqueue_pk(lg_ctx* c, int tok, int pos)
{
    PkParams& P = c->pk;
    PkStep S = {};
    S.tok = tok; S.pos = pos; S.base = c->pk_base;
    S.trace = c->pk_trace;
    S.act_trace = c->act_trace;
    c->pk_trace = nullptr;   /* one step only */
    c->act_trace = nullptr;
    int rc = lg_persist_launch(c->pk_kernel, c->pk, &S, c->pk_nwg, c->stream);
    if (rc) return rc;
    c->pk_base += 5ull * c->n_layers + 1;
    LG_HIP_CHECK(hipMemcpyAsync(c->pk_status_host, P.tok_out, 2 * sizeof(int), hipMemcpyDeviceToHost, c->stream));
    c->last_was_pk = true;
    return LG_OK;
}

/* after a synchronize: turn an expired wait of the last persistent step
 * into an error (and reset the counters for the next step) */
static int pk_check(lg_ctx* c)
{
    c->ring_pending = 0;
    if (!c->last_was_pk || !c->pk_status_host) return LG_OK;
    if (use_fused(c)) {
        /* the output kernel advanced the step record to {token, pos + 1} */
        c->dev_tok = c->pk_status_host[0];
        c->dev_pos = c->last_pos + 1;
        c->dev_known = true;
    }
    if (c->pk_status_host[1]) {
        const int code = c->pk_status_host[1];
        pk_reset(c);
        c->pk_status_host[1] = 0;
        lg_set_error(code == 1 ? "persistent decode: a workgroup sync wait expired"
                               : "persistent decode: unsupported phase configuration");
        return LG_ERR_STATE;
    }
    return LG_OK;
}

extern "C" int lg_set_decode_path(lg_ctx* ctx, int path)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    if (path != LG_PATH_AUTO && path != LG_PATH_PERSISTENT && path != LG_PATH_MULTI && path != LG_PATH_FUSED) {
        lg_set_error("lg_set_decode_path: unknown path %d", path);
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    if (path == LG_PATH_FUSED && !(ctx->pk_ok && ctx->fused_fn)) {
        lg_set_error("lg_set_decode_path: the loaded model is not supported by the fused kernels");
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    if (path == LG_PATH_PERSISTENT && !(ctx->pk_ok && ctx->pk_kernel)) {
        lg_set_error("lg_set_decode_path: the loaded model is not supported by the persistent kernel");
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    ctx->path = path;
    return LG_OK;
}

extern "C" int lg_trace_next_step(lg_ctx* ctx, uint64_t* trace_dev)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    ctx->pk_trace = trace_dev;
    return LG_OK;
}

extern "C" int lg_trace_acts_next_step(lg_ctx* ctx, void* trace_dev)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    ctx->act_trace = (uint8_t*)trace_dev;
    return LG_OK;
}

extern "C" int lg_trace_acts_next_prefill(lg_ctx* ctx, void* trace_dev)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    ctx->pf_trace = (uint8_t*)trace_dev;
    return LG_OK;
}

extern "C" size_t lg_trace_acts_size(const lg_ctx* ctx)
{
    if (!ctx || !ctx->loaded) return 0;
    return (size_t)(4 * ctx->n_layers + 1) * ctx->act_stride;
}

extern "C" size_t lg_trace_size(const lg_ctx* ctx)
{
    if (!ctx || !ctx->pk_ok) return 0;
    return (size_t)(5 * ctx->n_layers + 1) * ctx->pk_nwg * 4 * sizeof(uint64_t);
}

extern "C" int lg_hbm_read_probe(const void* buf, size_t bytes, int iters, float* avg_us, void* stream)
{
    if (iters <= 0 || !avg_us) { lg_set_error("lg_hbm_read_probe: bad arguments"); return LG_ERR_ARG; }
    hipStream_t s = (hipStream_t)stream;
    int rc = lg_launch_read_probe(buf, bytes, s);   /* untimed first pass */
    if (rc) return rc;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    LG_HIP_CHECK(hipEventCreate(&e0));
    LG_HIP_CHECK(hipEventCreate(&e1));
    hipEventRecord(e0, s);
    for (int i = 0; i < iters && !rc; i++) rc = lg_launch_read_probe(buf, bytes, s);
    hipEventRecord(e1, s);
    const hipError_t e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (!rc && e == hipSuccess) hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc) return rc;
    if (e != hipSuccess) { lg_set_error("lg_hbm_read_probe: %s", hipGetErrorString(e)); return LG_ERR_HIP; }
    *avg_us = ms * 1e3f / (float)iters;
    return LG_OK;
}

extern "C" int lg_time_fused_phase(lg_ctx* ctx, int phase, int layer0, int iters, float* avg_us)
{
    if (!ctx || !avg_us || iters <= 0 || phase < 0 || phase > 5 || layer0 < 0) {
        lg_set_error("time_fused_phase: bad argument");
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    if (!ctx->loaded || !use_fused(ctx)) {
        lg_set_error("time_fused_phase: the fused decode path is not in use");
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    /* the kernels read the device step record: it must hold a known position */
    if (!ctx->dev_known || ctx->dev_pos >= ctx->n_context) {
        lg_set_error("time_fused_phase: run and synchronize a decode step first");
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    hipEvent_t e0, e1;
    LG_HIP_CHECK(hipEventCreate(&e0));
    LG_HIP_CHECK(hipEventCreate(&e1));
    LG_HIP_CHECK(hipEventRecord(e0, ctx->stream));
    int rc = LG_OK;
    for (int i = 0; i < iters && rc == LG_OK; i++)
        rc = lg_fused_phase(ctx->fused_fn, ctx->pk, ctx->pk_layers.data(), ctx->step_dev, phase,
                            (layer0 + i) % ctx->n_layers, ctx->pk_nwg, att_long(ctx, ctx->dev_pos), ctx->stream);
    LG_HIP_CHECK(hipEventRecord(e1, ctx->stream));
    LG_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    LG_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    /* the output-head kernel advances the step record: rewrite it before the next step */
    if (phase == 5) ctx->dev_known = false;
    if (rc) return ctx_fail(ctx, rc);
    *avg_us = ms * 1000.0f / (float)iters;
    return LG_OK;
}

extern "C" int lg_decode_path(const lg_ctx* ctx)
{
    if (!ctx || !ctx->loaded) return -1;
    return use_pk(ctx) ? LG_PATH_PERSISTENT : (use_fused(ctx) ? LG_PATH_FUSED : LG_PATH_MULTI);
}

/* ------------------------------------------------------------------ */
/* batched prefill set-up                                               */
/* ------------------------------------------------------------------ */
#define LG_PF_TMAX 512   /* tokens per layer pass */

/* the batched prefill serves models whose layer matrices all have a batched
 * GEMM (the K-quants, Q8_0, Q1_0, Q1_G on int8 MFMA, F32/F16 on fp32 MFMA;
 * any mix, Q|K|V and up|gate stacked or not) and whose attention shape the
 * prefill attention kernel takes */
static PfMat pf_mat(const dweight& w) { return PfMat{w.data, w.rsz, w.type, w.rows}; }

static void setup_prefill(lg_ctx* ctx, const lg_model_desc* m)
{
    ctx->pf_ok = false;
    ctx->pf_fam = 0;
    bool ok = lg_prefill_attn_supported(m->head_dim, m->n_heads / m->n_kv_heads) && !ctx->layers.empty();
    int fam = 0;
    auto take = [&](const dweight& w) {
        const int at = lg_prefill_act_type(w.type);
        /* the Q1_G GEMM steps 256 values */
        if (at < 0 || (w.type == LG_Q1_G && w.cols % 256)) ok = false;
        fam |= at == LG_Q8_K ? 1 : at == LG_Q8_0 ? 2 : 4;
    };
    for (int l = 0; ok && l < m->n_layers; l++) {
        const dlayer& D = ctx->layers[l];
        if (D.qkv_fused) take(D.qkv);
        else { take(D.q); take(D.k); take(D.v); }
        take(D.att_out);
        if (D.ug_fused) take(D.ug);
        else { take(D.up); take(D.gate); }
        take(D.down);
        ok = ok && D.down.cols == m->n_ff;
    }
    if (!ok) return;
    ctx->pf_layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        const dlayer& D = ctx->layers[l];
        PfLayer& L = ctx->pf_layers[l];
        L = PfLayer{};
        L.qkv_fused = D.qkv_fused;
        L.ug_fused = D.ug_fused;
        if (D.qkv_fused) L.qkv = pf_mat(D.qkv);
        else { L.q = pf_mat(D.q); L.k = pf_mat(D.k); L.v = pf_mat(D.v); }
        L.ao = pf_mat(D.att_out);
        if (D.ug_fused) L.ug = pf_mat(D.ug);
        else { L.up = pf_mat(D.up); L.gate = pf_mat(D.gate); }
        L.down = pf_mat(D.down);
        if (ctx->pk_ok && l < (int)ctx->pk_layers.size()) {
            /* matrices the fused step reads from regrouped copies (uniform
             * Q8_0 / Q1_0 / Q6_K layers, a mixed layer's Q6_K V and down):
             * the batched GEMMs read those too (aligned 16-byte loads, the
             * same values) */
            const PkLayer& K = ctx->pk_layers[l];
            const bool k32 = !lg_prefill_gemm16();   /* the 16 x 16 Q6_K and Q1_G kernels read GGUF rows only */
            auto rep = [&](PfMat& M, const uint8_t* w, int t) {
                if ((M.type == LG_Q8_0 && t == LG_Q8_0_R) || (M.type == LG_Q1_0 && t == LG_Q1_0_R) ||
                    (k32 && M.type == LG_Q6_K && t == LG_Q6_K_R) || (k32 && M.type == LG_Q1_G && t == LG_Q1_G_R)) {
                    M.w = w;
                    M.type = t;
                }
            };
            if (D.qkv_fused) rep(L.qkv, K.qkv, K.qkv_t);
            else if (D.qk_fused && K.v) rep(L.v, K.v, K.v_t);
            rep(L.ao, K.ao, K.ao_t);
            if (D.ug_fused) rep(L.ug, K.ug, K.ug_t);
            rep(L.down, K.down, K.down_t);
        }
        L.att_norm = D.att_norm; L.ffn_norm = D.ffn_norm; L.q_norm = D.q_norm; L.k_norm = D.k_norm;
    }
    PfModel& M = ctx->pf_model;
    M.layers = ctx->pf_layers.data();
    M.n_layers = m->n_layers; M.n_embed = m->n_embed; M.n_heads = m->n_heads; M.n_kv = m->n_kv_heads;
    M.head_dim = m->head_dim; M.kv_dim = m->kv_dim; M.n_ff = m->n_ff; M.n_ctx = m->n_context;
    M.rope_dim = m->rope_dim; M.eps = m->rms_epsilon;
    M.embd = ctx->embd.data; M.embd_rsz = ctx->embd.rsz; M.embd_t = ctx->embd.type;
    M.rope_freq = ctx->rope_freq; M.kc = ctx->kc; M.vc = ctx->vc;
    ctx->pf_fam = fam;
    ctx->pf_ok = true;
}

/* buffers for LG_PF_TMAX tokens, allocated at the first batched prefill:
 * the activation forms the model's matrices take, width up to
 * max(n_embed, n_ff) */
static int prefill_buffers(lg_ctx* c)
{
    if (c->pf.tmax) return LG_OK;
    PfBuffers B = {};
    const int tmax = std::min(LG_PF_TMAX, (c->n_context + 3) / 4 * 4);
    const size_t ne = c->n_embed, qs = ne + 2 * (size_t)c->kv_dim, nff = c->n_ff, wide = std::max(ne, nff);
    int rc;
    if ((rc = dalloc(c, (void**)&B.toks, (size_t)tmax * sizeof(int)))) return rc;
    if ((rc = dalloc(c, (void**)&B.x, (size_t)tmax * ne * 4))) return rc;
    if ((rc = dalloc(c, (void**)&B.qkv, (size_t)tmax * qs * 4))) return rc;
    if ((rc = dalloc(c, (void**)&B.att, (size_t)tmax * ne * 4))) return rc;
    if ((rc = dalloc(c, (void**)&B.ug, (size_t)tmax * 2 * nff * 4))) return rc;
    if (c->pf_fam & 1) {   /* Q8_K: quants, a scale and 16 bsums per 256 values */
        if ((rc = dalloc(c, (void**)&B.qk.qs, (size_t)tmax * wide))) return rc;
        if ((rc = dalloc(c, (void**)&B.qk.d, wide / 256 * tmax * 4))) return rc;
        if ((rc = dalloc(c, (void**)&B.qk.bs, (size_t)tmax * (wide / 256) * 16 * 2))) return rc;
        B.qk.tld = tmax;
    }
    if (c->pf_fam & 4) {   /* F32/F16 weights: the fp32 activations */
        if ((rc = dalloc(c, (void**)&B.qf.f, (size_t)tmax * wide * 4))) return rc;
        B.qf.tld = tmax;
    }
    if (c->pf_fam & 2) {   /* Q8_0: quants, a scale and a sum per 32 values */
        if ((rc = dalloc(c, (void**)&B.q0.qs, (size_t)tmax * wide))) return rc;
        if ((rc = dalloc(c, (void**)&B.q0.d, wide / 32 * tmax * 4))) return rc;
        if ((rc = dalloc(c, (void**)&B.q0.as, wide / 32 * tmax * 4))) return rc;
        B.q0.tld = tmax;
    }
    B.tmax = tmax;
    c->pf = B;
    return LG_OK;
}

static int load_model_impl(lg_ctx* ctx, const lg_model_desc* m)
{
    if (!m || !m->layers) { lg_set_error("load_model: null descriptor"); return LG_ERR_ARG; }
    if (m->arch != LG_ARCH_LLAMA && m->arch != LG_ARCH_QWEN3) { lg_set_error("load_model: arch %d unsupported", m->arch); return LG_ERR_ARG; }
    if (m->n_layers <= 0 || m->n_embed <= 0 || m->n_heads <= 0 || m->n_kv_heads <= 0 || m->head_dim <= 0 ||
        m->n_ff <= 0 || m->vocab_size <= 0 || m->n_context <= 0 || m->n_heads % m->n_kv_heads ||
        m->kv_dim != m->n_kv_heads * m->head_dim || m->n_heads * m->head_dim != m->n_embed) {
        /* q and the attention output are n_embed wide in the reference
         * (fast/common.cpp:28, fast/ligguf_fast_qk.cpp:40,109) */
        lg_set_error("load_model: inconsistent dimensions");
        return LG_ERR_ARG;
    }
    if (m->n_embed % 32 || m->n_ff % 32 || m->head_dim % 4 || m->head_dim > 256) {
        lg_set_error("load_model: n_embed/n_ff must be multiples of 32 and head_dim a multiple of 4 up to 256");
        return LG_ERR_ARG;
    }
    if (m->rope_dim > 0 && !m->rope_freq) { lg_set_error("load_model: rope_freq missing"); return LG_ERR_ARG; }
    int rc;
    if ((rc = check_weight(m->token_embd, m->token_embd.rows, m->n_embed, "token_embd"))) return rc;
    if ((rc = check_weight(m->output, m->vocab_size, m->n_embed, "output"))) return rc;
    for (int l = 0; l < m->n_layers; l++) {
        const lg_layer_desc& L = m->layers[l];
        if ((rc = check_weight(L.att_q, m->n_embed, m->n_embed, "attn_q"))) return rc;
        if ((rc = check_weight(L.att_k, m->kv_dim, m->n_embed, "attn_k"))) return rc;
        if ((rc = check_weight(L.att_v, m->kv_dim, m->n_embed, "attn_v"))) return rc;
        if ((rc = check_weight(L.att_out, m->n_embed, m->n_embed, "attn_output"))) return rc;
        if ((rc = check_weight(L.ffn_up, m->n_ff, m->n_embed, "ffn_up"))) return rc;
        if ((rc = check_weight(L.ffn_gate, m->n_ff, m->n_embed, "ffn_gate"))) return rc;
        if ((rc = check_weight(L.ffn_down, m->n_embed, m->n_ff, "ffn_down"))) return rc;
        if (!L.att_norm || !L.ffn_norm) { lg_set_error("load_model: layer %d norms missing", l); return LG_ERR_ARG; }
        if (m->arch == LG_ARCH_QWEN3 && (!L.att_q_norm || !L.att_k_norm)) { lg_set_error("load_model: layer %d QK norms missing", l); return LG_ERR_ARG; }
    }
    /* K-quant activations need 256-wide blocks (quantize_q8_K asserts it,
     * fast/lil_math.cpp:360) */
    auto needs_k = [&](int n, int t) { return act_family(t) == ACT_K && n % 256; };
    for (int l = 0; l < m->n_layers; l++) {
        const lg_layer_desc& L = m->layers[l];
        if (needs_k(m->n_embed, L.att_q.type) || needs_k(m->n_embed, L.att_k.type) || needs_k(m->n_embed, L.att_v.type) ||
            needs_k(m->n_embed, L.att_out.type) || needs_k(m->n_embed, L.ffn_up.type) ||
            needs_k(m->n_embed, L.ffn_gate.type) || needs_k(m->n_ff, L.ffn_down.type)) {
            lg_set_error("load_model: K-quant weights need widths that are multiples of 256");
            return LG_ERR_ARG;
        }
    }

    free_model(ctx);
    ctx->arch = m->arch; ctx->n_layers = m->n_layers; ctx->n_embed = m->n_embed; ctx->n_heads = m->n_heads;
    ctx->n_kv_heads = m->n_kv_heads; ctx->head_dim = m->head_dim; ctx->kv_dim = m->kv_dim; ctx->n_ff = m->n_ff;
    ctx->vocab = m->vocab_size; ctx->n_context = m->n_context; ctx->rope_dim = m->rope_dim; ctx->eps = m->rms_epsilon;
    {
        /* activation trace slot: the widest quantized vector in either form */
        const int64_t wide = std::max(m->n_embed, m->n_ff);
        const int64_t qk = std::max<int64_t>(lg_row_size(LG_Q8_K, wide / 256 * 256), 0);
        const int64_t q0 = std::max<int64_t>(lg_row_size(LG_Q8_0, wide / 32 * 32), 0);
        ctx->act_stride = (size_t)((std::max(qk, q0) + 255) / 256 * 256);
    }

    if ((rc = upload_weight(ctx, m->token_embd, ctx->embd))) return rc;
    if ((rc = upload_weight(ctx, m->output, ctx->output))) return rc;
    if ((rc = upload_floats(ctx, m->output_norm, m->n_embed, &ctx->out_norm, "output_norm"))) return rc;
    {
        /* rope table padded with zeros to at least head_dim floats: the
         * whole-step attention loads a fixed slice per lane */
        const int nfreq = m->rope_dim / 2 > 0 ? m->rope_dim / 2 : 0;
        const size_t nalloc = std::max<size_t>((size_t)std::max(nfreq, m->head_dim), 1);
        std::vector<float> tab(nalloc, 0.0f);
        if (nfreq) std::copy(m->rope_freq, m->rope_freq + nfreq, tab.begin());
        if ((rc = upload_floats(ctx, tab.data(), nalloc, &ctx->rope_freq, "rope_freq"))) return rc;
    }
    {
        /* one shape and type per matrix kind over all layers, Q|K|V and
         * up|gate stackable: one allocation per kind */
        const lg_layer_desc& L0 = m->layers[0];
        auto same = [](const lg_weight& a, const lg_weight& b) {
            return a.type == b.type && a.rsz == b.rsz && a.rows == b.rows && a.cols == b.cols;
        };
        bool uni = L0.att_q.type == L0.att_k.type && L0.att_q.type == L0.att_v.type && L0.att_q.rsz == L0.att_k.rsz &&
                   L0.att_q.rsz == L0.att_v.rsz && L0.ffn_up.type == L0.ffn_gate.type && L0.ffn_up.rsz == L0.ffn_gate.rsz;
        for (int l = 1; uni && l < m->n_layers; l++) {
            const lg_layer_desc& L = m->layers[l];
            uni = same(L.att_q, L0.att_q) && same(L.att_k, L0.att_k) && same(L.att_v, L0.att_v) &&
                  same(L.att_out, L0.att_out) && same(L.ffn_up, L0.ffn_up) && same(L.ffn_gate, L0.ffn_gate) &&
                  same(L.ffn_down, L0.ffn_down);
        }
        auto& A = ctx->arena;
        A = {};
        if (uni) {
            const size_t nl = m->n_layers;
            A.qkv_b = (size_t)(L0.att_q.rows + L0.att_k.rows + L0.att_v.rows) * L0.att_q.rsz;
            A.ao_b = (size_t)L0.att_out.rows * L0.att_out.rsz;
            A.ug_b = (size_t)(L0.ffn_up.rows + L0.ffn_gate.rows) * L0.ffn_up.rsz;
            A.down_b = (size_t)L0.ffn_down.rows * L0.ffn_down.rsz;
            if ((rc = dalloc(ctx, (void**)&A.qkv, nl * A.qkv_b))) return rc;
            if ((rc = dalloc(ctx, (void**)&A.ao, nl * A.ao_b))) return rc;
            if ((rc = dalloc(ctx, (void**)&A.ug, nl * A.ug_b))) return rc;
            if ((rc = dalloc(ctx, (void**)&A.down, nl * A.down_b))) return rc;
            if ((rc = dalloc(ctx, (void**)&A.att_norm, nl * m->n_embed * 4))) return rc;
            if ((rc = dalloc(ctx, (void**)&A.ffn_norm, nl * m->n_embed * 4))) return rc;
            if (m->arch == LG_ARCH_QWEN3) {
                if ((rc = dalloc(ctx, (void**)&A.q_norm, nl * m->head_dim * 4))) return rc;
                if ((rc = dalloc(ctx, (void**)&A.k_norm, nl * m->head_dim * 4))) return rc;
            }
            A.ok = true;
        }
    }
    const auto& AR = ctx->arena;
    auto slot = [&](uint8_t* base, size_t stride, int l) { return base ? base + (size_t)l * stride : nullptr; };
    auto fslot = [&](float* base, size_t stride, int l) { return base ? base + (size_t)l * stride : nullptr; };
    ctx->layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        const lg_layer_desc& L = m->layers[l];
        dlayer& D = ctx->layers[l];
        if ((rc = upload_floats(ctx, L.att_norm, m->n_embed, &D.att_norm, "attn_norm", fslot(AR.att_norm, m->n_embed, l))))
            return rc;
        if ((rc = upload_floats(ctx, L.ffn_norm, m->n_embed, &D.ffn_norm, "ffn_norm", fslot(AR.ffn_norm, m->n_embed, l))))
            return rc;
        if (m->arch == LG_ARCH_QWEN3) {
            if ((rc = upload_floats(ctx, L.att_q_norm, m->head_dim, &D.q_norm, "attn_q_norm",
                                    fslot(AR.q_norm, m->head_dim, l))))
                return rc;
            if ((rc = upload_floats(ctx, L.att_k_norm, m->head_dim, &D.k_norm, "attn_k_norm",
                                    fslot(AR.k_norm, m->head_dim, l))))
                return rc;
        }
        if (L.att_q.type == L.att_k.type && L.att_q.type == L.att_v.type && L.att_q.rsz == L.att_k.rsz &&
            L.att_q.rsz == L.att_v.rsz) {
            const lg_weight* ws[3] = {&L.att_q, &L.att_k, &L.att_v};
            dweight views[3];
            if ((rc = upload_stacked(ctx, ws, 3, D.qkv, views, slot(AR.qkv, AR.qkv_b, l)))) return rc;
            D.q = views[0]; D.k = views[1]; D.v = views[2];
            D.qkv_fused = true;
        } else if (L.att_q.type == L.att_k.type && L.att_q.rsz == L.att_k.rsz) {
            /* a Q4_K_M-style V of its own type: Q|K still one matrix */
            const lg_weight* ws[2] = {&L.att_q, &L.att_k};
            dweight views[2];
            if ((rc = upload_stacked(ctx, ws, 2, D.qkv, views, nullptr))) return rc;
            D.q = views[0]; D.k = views[1];
            if ((rc = upload_weight(ctx, L.att_v, D.v))) return rc;
            D.qk_fused = true;
        } else {
            if ((rc = upload_weight(ctx, L.att_q, D.q))) return rc;
            if ((rc = upload_weight(ctx, L.att_k, D.k))) return rc;
            if ((rc = upload_weight(ctx, L.att_v, D.v))) return rc;
        }
        if ((rc = upload_weight(ctx, L.att_out, D.att_out, slot(AR.ao, AR.ao_b, l)))) return rc;
        if (L.ffn_up.type == L.ffn_gate.type && L.ffn_up.rsz == L.ffn_gate.rsz) {
            const lg_weight* ws[2] = {&L.ffn_up, &L.ffn_gate};
            dweight views[2];
            if ((rc = upload_stacked(ctx, ws, 2, D.ug, views, slot(AR.ug, AR.ug_b, l)))) return rc;
            D.up = views[0]; D.gate = views[1];
            D.ug_fused = true;
        } else {
            if ((rc = upload_weight(ctx, L.ffn_up, D.up))) return rc;
            if ((rc = upload_weight(ctx, L.ffn_gate, D.gate))) return rc;
        }
        if ((rc = upload_weight(ctx, L.ffn_down, D.down, slot(AR.down, AR.down_b, l)))) return rc;
    }

    const size_t kvn = (size_t)m->n_layers * m->n_context * m->kv_dim;
    if ((rc = dalloc(ctx, (void**)&ctx->kc, kvn * 2))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->vc, kvn * 2))) return rc;
    LG_HIP_CHECK(hipMemset(ctx->kc, 0, kvn * 2));
    LG_HIP_CHECK(hipMemset(ctx->vc, 0, kvn * 2));

    const int wide = m->n_ff > m->n_embed ? m->n_ff : m->n_embed;
    if ((rc = dalloc(ctx, (void**)&ctx->x, (size_t)m->n_embed * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->qkv, (size_t)(m->n_embed + 2 * m->kv_dim) * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->att, (size_t)m->n_embed * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->hb, (size_t)2 * m->n_ff * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->logits, (size_t)m->vocab_size * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->xf, (size_t)wide * 4))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->xqk, (size_t)(wide / 256 + 1) * LG_BS_Q8_K))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->xq0, (size_t)(wide / 32 + 8) * LG_BS_Q8_0))) return rc;
    ctx->attn_ws_bytes = lg_attn_ws_bytes(m->n_heads, m->head_dim, m->n_context - 1);
    if ((rc = dalloc(ctx, (void**)&ctx->attn_ws, ctx->attn_ws_bytes))) return rc;
    if ((rc = dalloc(ctx, (void**)&ctx->argmax_dev, 16))) return rc;
    if ((rc = setup_persistent(ctx, m))) return rc;
    setup_prefill(ctx, m);
    LG_HIP_CHECK(hipDeviceSynchronize());
    ctx->loaded = true;
    return LG_OK;
}

extern "C" int lg_load_model(lg_ctx* ctx, const lg_model_desc* desc)
{
    if (!ctx) { lg_set_error("lg_load_model: null context"); return LG_ERR_ARG; }
    lg_rand_guard keep_rand;
    hipSetDevice(ctx->device);
    int rc;
    {
        lg_uploader up;
        rc = up.init(ctx->stream);
        if (!rc) {
            g_up = &up;
            rc = load_model_impl(ctx, desc);
            g_up = nullptr;
            if (!rc) rc = up.finish();
        }
    }
    if (rc) free_model(ctx);
    return ctx_fail(ctx, rc);
}

/* ------------------------------------------------------------------ */
/* the step                                                             */
/* ------------------------------------------------------------------ */

/* quantized forms of the activation for the weights in `fam` */
struct actbufs {
    const void* k;
    const void* q0;
    const float* f;
};

static int prep_norm(lg_ctx* c, const float* x, const float* w, int n, int fam, actbufs& a)
{
    int rc;
    a.k = c->xqk; a.q0 = c->xq0; a.f = c->xf;
    if (fam & ACT_K) if ((rc = lg_launch_rmsnorm_quant(x, w, n, c->eps, LG_Q8_K, c->xqk, (fam & ACT_F) ? c->xf : nullptr, c->stream))) return rc;
    if (fam & ACT_80) if ((rc = lg_launch_rmsnorm_quant(x, w, n, c->eps, LG_Q8_0, c->xq0, (fam & ACT_F) && !(fam & ACT_K) ? c->xf : nullptr, c->stream))) return rc;
    if (fam == ACT_F) if ((rc = lg_launch_rmsnorm_quant(x, w, n, c->eps, LG_F32, nullptr, c->xf, c->stream))) return rc;
    return LG_OK;
}

static int prep_plain(lg_ctx* c, const float* x, int n, int fam, actbufs& a)
{
    int rc;
    a.k = c->xqk; a.q0 = c->xq0; a.f = x;
    if (fam & ACT_K) if ((rc = lg_launch_quantize_q8_K(x, n, c->xqk, c->stream))) return rc;
    if (fam & ACT_80) if ((rc = lg_launch_quantize_q8_0(x, n, c->xq0, c->stream))) return rc;
    return LG_OK;
}

static const void* act_for(const actbufs& a, int type)
{
    const int f = act_family(type);
    return f == ACT_K ? a.k : (f == ACT_80 ? a.q0 : (const void*)a.f);
}

static int mv(lg_ctx* c, const dweight& w, const actbufs& a, float* out, int acc)
{
    return lg_launch_matvec(w.type, w.data, w.rsz, w.cols, w.rows, act_for(a, w.type), out, acc, c->stream);
}

/* activation trace of the multi-kernel step: the quantized form of an
 * activation of width n that the weights of family `fam` read (Q8_K when
 * any of them takes it, else Q8_0), copied to slot k */
static int trace_act(lg_ctx* c, uint8_t* tr, int k, int fam, int n)
{
    if (!tr || !(fam & (ACT_K | ACT_80))) return LG_OK;
    const bool kq = (fam & ACT_K) != 0;
    const int64_t bytes = lg_row_size(kq ? LG_Q8_K : LG_Q8_0, n);
    if (bytes <= 0) return LG_OK;
    LG_HIP_CHECK(hipMemcpyAsync(tr + (size_t)k * c->act_stride, kq ? c->xqk : c->xq0, (size_t)bytes,
                                hipMemcpyDeviceToDevice, c->stream));
    return LG_OK;
}

static int enqueue_step(lg_ctx* c, int tok, int pos)
{
    if (use_pk(c)) return enqueue_pk(c, tok, pos);
    if (use_fused(c)) return enqueue_fused(c, tok, pos);
    c->last_was_pk = false;
    uint8_t* atr = c->act_trace;   /* one step only */
    c->act_trace = nullptr;
    int rc;
    const int ne = c->n_embed, kvd = c->kv_dim;
    float* q = c->qkv;
    float* k = c->qkv + ne;
    float* v = c->qkv + ne + kvd;
    if ((rc = lg_launch_embed(c->embd.type, c->embd.data, c->embd.rsz, nullptr, tok, ne, c->x, c->stream))) return rc;
    for (int l = 0; l < c->n_layers; l++) {
        const dlayer& L = c->layers[l];
        actbufs a;
        /* attention branch */
        const int fam_qkv = act_family(L.q.type) | act_family(L.k.type) | act_family(L.v.type);
        if ((rc = prep_norm(c, c->x, L.att_norm, ne, fam_qkv, a))) return rc;
        if ((rc = trace_act(c, atr, 4 * l, fam_qkv, ne))) return rc;
        if (L.qkv_fused) {
            if ((rc = mv(c, L.qkv, a, c->qkv, 0))) return rc;
        } else {
            if ((rc = mv(c, L.q, a, q, 0))) return rc;
            if ((rc = mv(c, L.k, a, k, 0))) return rc;
            if ((rc = mv(c, L.v, a, v, 0))) return rc;
        }
        const size_t loff = (size_t)l * c->n_context * kvd;
        uint16_t* kc = c->kc + loff;
        uint16_t* vc = c->vc + loff;
        if ((rc = lg_launch_qk_norm_rope_kv(q, k, v, L.q_norm, L.k_norm, c->n_heads, c->n_kv_heads, c->head_dim,
                                            c->rope_dim, pos, c->rope_freq, c->eps, kc + (size_t)pos * kvd,
                                            vc + (size_t)pos * kvd, c->stream)))
            return rc;
        if ((rc = lg_launch_attn(q, k, v, kc, vc, c->n_heads, c->n_kv_heads, c->head_dim, pos, c->att, c->attn_ws,
                                 c->attn_ws_bytes, c->stream)))
            return rc;
        if ((rc = prep_plain(c, c->att, ne, act_family(L.att_out.type), a))) return rc;
        if ((rc = trace_act(c, atr, 4 * l + 1, act_family(L.att_out.type), ne))) return rc;
        if ((rc = mv(c, L.att_out, a, c->x, 1))) return rc;
        /* FFN branch */
        const int fam_ug = act_family(L.up.type) | act_family(L.gate.type);
        if ((rc = prep_norm(c, c->x, L.ffn_norm, ne, fam_ug, a))) return rc;
        if ((rc = trace_act(c, atr, 4 * l + 2, fam_ug, ne))) return rc;
        float* hb = c->hb;
        float* hb2 = c->hb + c->n_ff;
        if (L.ug_fused) {
            if ((rc = mv(c, L.ug, a, hb, 0))) return rc;
        } else {
            if ((rc = mv(c, L.up, a, hb, 0))) return rc;
            if ((rc = mv(c, L.gate, a, hb2, 0))) return rc;
        }
        const int fam_d = act_family(L.down.type);
        if (fam_d == ACT_K) {
            if ((rc = lg_launch_swiglu_quant(hb, hb2, c->n_ff, LG_Q8_K, c->xqk, c->stream))) return rc;
        } else if (fam_d == ACT_80) {
            if ((rc = lg_launch_swiglu_quant(hb, hb2, c->n_ff, LG_Q8_0, c->xq0, c->stream))) return rc;
        } else {
            if ((rc = lg_launch_swiglu_quant(hb, hb2, c->n_ff, LG_F32, nullptr, c->stream))) return rc;
        }
        a.k = c->xqk; a.q0 = c->xq0; a.f = hb;
        if ((rc = trace_act(c, atr, 4 * l + 3, fam_d, c->n_ff))) return rc;
        if ((rc = mv(c, L.down, a, c->x, 1))) return rc;
    }
    actbufs a;
    if ((rc = prep_norm(c, c->x, c->out_norm, ne, act_family(c->output.type), a))) return rc;
    if ((rc = trace_act(c, atr, 4 * c->n_layers, act_family(c->output.type), ne))) return rc;
    if ((rc = mv(c, c->output, a, c->logits, 0))) return rc;
    return LG_OK;
}

static int step_checks(lg_ctx* ctx, int tok, int pos)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return LG_ERR_STATE; }
    if (pos < 0 || pos >= ctx->n_context) { lg_set_error("position %d outside the context of %d", pos, ctx->n_context); return LG_ERR_STATE; }
    if (tok < 0 || tok >= ctx->embd.rows) { lg_set_error("token %d outside the vocabulary of %d", tok, ctx->embd.rows); return LG_ERR_ARG; }
    return LG_OK;
}

extern "C" int lg_decode_step_async(lg_ctx* ctx, int tok, int pos)
{
    int rc = step_checks(ctx, tok, pos);
    if (rc) return ctx_fail(ctx, rc);
    hipSetDevice(ctx->device);
    return ctx_fail(ctx, enqueue_step(ctx, tok, pos));
}

extern "C" int lg_sync(lg_ctx* ctx)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        lg_set_error("stream synchronize: %s", hipGetErrorString(e));
        return ctx_fail(ctx, LG_ERR_HIP);
    }
    return ctx_fail(ctx, pk_check(ctx));
}

extern "C" const float* lg_logits_device(lg_ctx* ctx) { return ctx && ctx->loaded ? ctx->logits : nullptr; }

extern "C" int lg_decode_step(lg_ctx* ctx, int tok, int pos, float* logits_host)
{
    int rc = lg_decode_step_async(ctx, tok, pos);
    if (rc) return rc;
    if (logits_host) {
        const hipError_t e = hipMemcpyAsync(logits_host, ctx->logits, (size_t)ctx->vocab * 4, hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) { lg_set_error("logits copy: %s", hipGetErrorString(e)); return ctx_fail(ctx, LG_ERR_HIP); }
    }
    return lg_sync(ctx);
}

extern "C" int lg_argmax(lg_ctx* ctx, int* tok_out)
{
    if (!ctx || !tok_out) { lg_set_error("lg_argmax: null argument"); return LG_ERR_ARG; }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    if (ctx->last_was_pk) {
        /* the persistent step reduced the argmax already and its status
         * copy is queued behind it */
        const int rc = lg_sync(ctx);
        if (rc) return rc;
        *tok_out = ctx->pk_status_host[0];
        return LG_OK;
    }
    int rc = lg_launch_argmax(ctx->logits, ctx->vocab, ctx->argmax_dev, ctx->stream);
    if (rc) return ctx_fail(ctx, rc);
    const hipError_t e = hipMemcpyAsync(tok_out, ctx->argmax_dev, sizeof(int), hipMemcpyDeviceToHost, ctx->stream);
    if (e != hipSuccess) { lg_set_error("argmax copy: %s", hipGetErrorString(e)); return ctx_fail(ctx, LG_ERR_HIP); }
    return lg_sync(ctx);
}

extern "C" int lg_decode_greedy(lg_ctx* ctx, int tok, int pos, int n, int* toks_out)
{
    int rc = step_checks(ctx, tok, pos);
    if (rc) return ctx_fail(ctx, rc);
    if (n <= 0 || !toks_out || n > ctx->n_context - pos) {
        lg_set_error("lg_decode_greedy: %d steps from position %d (context %d), or no output", n, pos, ctx->n_context);
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    hipSetDevice(ctx->device);
    if (use_fused(ctx) || use_pk(ctx)) {
        /* whole-step paths: every step leaves its greedy token on the device
         * (the fused output kernel advances the step record; the persistent
         * kernel takes tok < 0 as the previous step's token) and in tok_hist */
        if (use_fused(ctx)) {
            if ((rc = fused_set_step(ctx, tok, pos, 0))) return ctx_fail(ctx, rc);
            for (int i = 0; i < n; i++)
                if ((rc = fused_launch(ctx, pos + i))) return ctx_fail(ctx, rc);
            ctx->last_pos = pos + n - 1;
        } else {
            for (int i = 0; i < n; i++)
                if ((rc = enqueue_pk(ctx, i ? -1 : tok, pos + i))) return ctx_fail(ctx, rc);
        }
        ctx->dev_known = false;
        LG_HIP_CHECK(hipMemcpyAsync(ctx->pk_status_host, ctx->pk.tok_out, 2 * sizeof(int), hipMemcpyDeviceToHost,
                                    ctx->stream));
        LG_HIP_CHECK(hipMemcpyAsync(toks_out, ctx->pk.tok_hist + pos, (size_t)n * sizeof(int), hipMemcpyDeviceToHost,
                                    ctx->stream));
        ctx->last_was_pk = true;
        return lg_sync(ctx);
    }
    /* the multi-kernel path: a step and its argmax at a time */
    for (int i = 0; i < n; i++) {
        if ((rc = lg_decode_step_async(ctx, tok, pos + i))) return rc;
        if ((rc = lg_argmax(ctx, &tok))) return rc;
        toks_out[i] = tok;
    }
    return LG_OK;
}

static int sample_args(float r01, const char* who)
{
    if (!(r01 >= 0.0f && r01 <= 1.0f)) {
        lg_set_error("%s: uniform draw %g outside [0, 1]", who, (double)r01);
        return LG_ERR_ARG;
    }
    return LG_OK;
}

extern "C" int lg_sample_topp(lg_ctx* ctx, float temp, float topp, int topk, float r01, int* tok_out)
{
    if (!ctx || !tok_out) { lg_set_error("lg_sample_topp: null argument"); return LG_ERR_ARG; }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    if (!(temp > 0.0f)) return lg_argmax(ctx, tok_out);   /* the reference's temp <= 0 case */
    int rc = sample_args(r01, "lg_sample_topp");
    if (rc) return rc;
    if (ctx->samp && lg_sample_ws_size(ctx->samp) != ctx->vocab) {
        LG_HIP_CHECK(hipStreamSynchronize(ctx->stream));
        lg_sample_ws_free(ctx->samp);
        ctx->samp = nullptr;
    }
    if (!ctx->samp && (rc = lg_sample_ws_alloc(ctx->vocab, &ctx->samp))) return ctx_fail(ctx, rc);
    if ((rc = lg_launch_sample_topp(ctx->logits, ctx->samp, temp, topp, topk, r01, ctx->stream))) return ctx_fail(ctx, rc);
    if ((rc = lg_sync(ctx))) return rc;
    *tok_out = *(volatile int*)lg_sample_ws_out_host(ctx->samp);
    if (*tok_out < 0) {
        lg_set_error("sampler: a workgroup did not publish its entries in time");
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    return LG_OK;
}

extern "C" int lg_sample_topp_device(const float* logits_dev, int n, float temp, float topp, int topk, float r01,
                                     int* tok_out)
{
    if (!logits_dev || !tok_out || n <= 0) { lg_set_error("lg_sample_topp_device: bad argument"); return LG_ERR_ARG; }
    int rc = sample_args(r01, "lg_sample_topp_device");
    if (rc) return rc;
    LgSampleWs* w = nullptr;
    if ((rc = lg_sample_ws_alloc(n, &w))) return rc;
    if (!(temp > 0.0f)) {
        rc = lg_launch_argmax(logits_dev, n, lg_sample_ws_out(w), nullptr);
        if (!rc) {
            const hipError_t e = hipMemcpy(tok_out, lg_sample_ws_out(w), sizeof(int), hipMemcpyDeviceToHost);
            if (e != hipSuccess) { lg_set_error("sample copy: %s", hipGetErrorString(e)); rc = LG_ERR_HIP; }
        }
    } else if (!(rc = lg_launch_sample_topp(logits_dev, w, temp, topp, topk, r01, nullptr))) {
        const hipError_t e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) { lg_set_error("sampler: %s", hipGetErrorString(e)); rc = LG_ERR_HIP; }
        else if ((*tok_out = *(volatile int*)lg_sample_ws_out_host(w)) < 0) {
            lg_set_error("sampler: a workgroup did not publish its entries in time");
            rc = LG_ERR_STATE;
        }
    }
    hipStreamSynchronize(nullptr);
    lg_sample_ws_free(w);
    return rc;
}

/* the prompt in layer passes of up to LG_PF_TMAX tokens (lg_prefill.hip),
 * then the output head on the last token's residual stream */
static int prefill_batched(lg_ctx* c, const int* toks, int n, int pos0)
{
    int rc;
    if ((rc = prefill_buffers(c))) return rc;
    LG_HIP_CHECK(hipStreamSynchronize(c->stream));   /* the token staging below reuses one buffer */
    /* a trace request covers every token of this prompt */
    uint8_t* tr = c->pf_trace;
    c->pf_trace = nullptr;
    const size_t tok_bytes = (size_t)(4 * c->n_layers + 1) * c->act_stride;
    c->pf.trace_stride = c->act_stride;
    int T = 0;
    for (int off = 0; off < n; off += T) {
        T = std::min(c->pf.tmax, n - off);
        c->pf.trace = tr ? tr + (size_t)off * tok_bytes : nullptr;
        LG_HIP_CHECK(hipMemcpyAsync(c->pf.toks, toks + off, (size_t)T * sizeof(int), hipMemcpyHostToDevice, c->stream));
        rc = lg_prefill_layers(c->pf_model, c->pf, T, pos0 + off, c->stream);
        c->pf.trace = nullptr;
        if (rc) return rc;
        if (off + T < n) LG_HIP_CHECK(hipStreamSynchronize(c->stream));
    }
    LG_HIP_CHECK(hipMemcpyAsync(c->x, c->pf.x + (size_t)(T - 1) * c->n_embed, (size_t)c->n_embed * 4,
                                hipMemcpyDeviceToDevice, c->stream));
    actbufs a;
    const int fam_o = act_family(c->output.type);
    if ((rc = prep_norm(c, c->x, c->out_norm, c->n_embed, fam_o, a))) return rc;
    if ((rc = trace_act(c, tr ? tr + (size_t)(n - 1) * tok_bytes : nullptr, 4 * c->n_layers, fam_o, c->n_embed))) return rc;
    if ((rc = mv(c, c->output, a, c->logits, 0))) return rc;
    c->last_was_pk = false;
    c->dev_known = false;
    return LG_OK;
}

extern "C" int lg_set_prefill_path(lg_ctx* ctx, int path)
{
    if (!ctx || path < LG_PREFILL_AUTO || path > LG_PREFILL_BATCHED) {
        lg_set_error("set_prefill_path: bad argument");
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    if (path == LG_PREFILL_BATCHED && ctx->loaded && !ctx->pf_ok) {
        lg_set_error("set_prefill_path: the batched prefill needs head_dim 48, 64 or 128 with 1, 2, 4 or 8 query "
                     "heads per KV head");
        return ctx_fail(ctx, LG_ERR_TYPE);
    }
    ctx->prefill_path = path;
    return LG_OK;
}

extern "C" int lg_prefill_path(const lg_ctx* ctx)
{
    if (!ctx || !ctx->loaded) return -1;
    return ctx->pf_ok && ctx->prefill_path != LG_PREFILL_STEPS ? LG_PREFILL_BATCHED : LG_PREFILL_STEPS;
}

extern "C" int lg_matmul_tokens(int type, const void* w, uint32_t rsz, int n, int d, const float* x, int T, float* out,
                                void* stream)
{
    const int at = lg_prefill_act_type(type);
    if (at < 0) {
        lg_set_error("matmul_tokens: type %d has no batched GEMM", type);
        return LG_ERR_TYPE;
    }
    if (!w || !x || !out || n <= 0 || n % (at == LG_Q8_K ? 256 : 32) || d <= 0 || T <= 0) {
        lg_set_error("matmul_tokens: bad arguments (n %d, d %d, T %d)", n, d, T);
        return LG_ERR_ARG;
    }
    if (at == LG_F32) {   /* fp32 activations as given */
        if (rsz != (uint32_t)n * (type == LG_F32 ? 4u : 2u)) {
            lg_set_error("matmul_tokens: row bytes %u for %d values", rsz, n);
            return LG_ERR_ARG;
        }
        int rc = lg_fgemm_tokens(type, (const uint8_t*)w, d, n, x, n, T, out, d, 0, (hipStream_t)stream);
        const hipError_t e2 = hipStreamSynchronize((hipStream_t)stream);
        if (!rc && e2 != hipSuccess) { lg_set_error("matmul_tokens: %s", hipGetErrorString(e2)); rc = LG_ERR_HIP; }
        return rc;
    }
    /* workspace: quants, then scales for n/32 blocks (enough for either
     * form), the Q8_K bsums and the Q8_0 sums */
    const int tld = (T + 3) / 4 * 4, nb = n / 256, nb0 = n / 32;
    PfQ8K q = {};
    q.tld = tld;
    const size_t o_d = (size_t)tld * n, o_bs = o_d + (size_t)nb0 * tld * 4, o_as = o_bs + (size_t)tld * nb * 32;
    const size_t bytes = o_as + (size_t)nb0 * tld * 4;
    uint8_t* ws = nullptr;
    const hipError_t e = hipMalloc((void**)&ws, bytes);
    if (e != hipSuccess) { lg_set_error("matmul_tokens: hipMalloc(%zu): %s", bytes, hipGetErrorString(e)); return LG_ERR_NOMEM; }
    q.qs = (int8_t*)ws;
    q.d = (float*)(ws + o_d);
    q.bs = (int16_t*)(ws + o_bs);
    q.as = (int*)(ws + o_as);
    int rc = lg_prefill_quantize(at, x, n, nullptr, 0.0f, n, T, q, (hipStream_t)stream);
    if (!rc) rc = lg_prefill_gemm(type, (const uint8_t*)w, rsz, d, n, q, T, out, d, 0, (hipStream_t)stream);
    const hipError_t e2 = hipStreamSynchronize((hipStream_t)stream);
    (void)hipFree(ws);
    if (!rc && e2 != hipSuccess) { lg_set_error("matmul_tokens: %s", hipGetErrorString(e2)); rc = LG_ERR_HIP; }
    return rc;
}

extern "C" int lg_prefill(lg_ctx* ctx, const int* toks, int n, int pos0, float* logits_host)
{
    if (!ctx || !toks || n <= 0) { lg_set_error("lg_prefill: bad arguments"); return ctx_fail(ctx, LG_ERR_ARG); }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    if (pos0 < 0 || pos0 + n > ctx->n_context) { lg_set_error("prefill of %d tokens at %d exceeds the context of %d", n, pos0, ctx->n_context); return ctx_fail(ctx, LG_ERR_STATE); }
    for (int i = 0; i < n; i++) {
        int rc = step_checks(ctx, toks[i], pos0 + i);
        if (rc) return ctx_fail(ctx, rc);
    }
    hipSetDevice(ctx->device);
    const bool batched = ctx->pf_ok && (ctx->prefill_path == LG_PREFILL_BATCHED ||
                                        (ctx->prefill_path == LG_PREFILL_AUTO && n >= 2));
    if (!batched) ctx->pf_trace = nullptr;   /* the prefill trace covers the batched path only */
    if (batched) {
        int rc = prefill_batched(ctx, toks, n, pos0);
        if (rc) return ctx_fail(ctx, rc);
    } else if (use_fused(ctx)) {
        /* the prompt goes to the device once; every replay of the step graph
         * takes its token from it (PkStep.feed_end) */
        LG_HIP_CHECK(hipStreamSynchronize(ctx->stream));   /* feed_host may back an earlier copy */
        ctx->ring_pending = 0;
        memcpy(ctx->feed_host + pos0, toks, (size_t)n * sizeof(int));
        LG_HIP_CHECK(hipMemcpyAsync(ctx->feed_dev + pos0, ctx->feed_host + pos0, (size_t)n * sizeof(int),
                                    hipMemcpyHostToDevice, ctx->stream));
        int rc = fused_set_step(ctx, toks[0], pos0, pos0 + n);
        for (int i = 0; !rc && i < n; i++) rc = fused_launch(ctx, pos0 + i);
        if (rc) return ctx_fail(ctx, rc);
        LG_HIP_CHECK(hipMemcpyAsync(ctx->pk_status_host, ctx->pk.tok_out, 2 * sizeof(int), hipMemcpyDeviceToHost,
                                    ctx->stream));
        ctx->dev_known = false;
        ctx->last_was_pk = true;
        ctx->last_pos = pos0 + n - 1;
    } else {
        for (int i = 0; i < n; i++) {
            int rc = enqueue_step(ctx, toks[i], pos0 + i);
            if (rc) return ctx_fail(ctx, rc);
        }
    }
    if (logits_host) {
        const hipError_t e = hipMemcpyAsync(logits_host, ctx->logits, (size_t)ctx->vocab * 4, hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) { lg_set_error("logits copy: %s", hipGetErrorString(e)); return ctx_fail(ctx, LG_ERR_HIP); }
    }
    return lg_sync(ctx);
}

static int kv_io(lg_ctx* ctx, int layer0, int nlayers, int pos0, int npos, uint16_t* kh, uint16_t* vh, bool write)
{
    if (!ctx) { lg_set_error("null context"); return LG_ERR_ARG; }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    if (layer0 < 0 || nlayers < 0 || layer0 + nlayers > ctx->n_layers || pos0 < 0 || npos < 0 ||
        pos0 + npos > ctx->n_context) {
        lg_set_error("kv range outside the cache");
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    hipSetDevice(ctx->device);
    const size_t row = (size_t)ctx->kv_dim * 2;
    for (int l = 0; l < nlayers; l++) {
        const size_t doff = ((size_t)(layer0 + l) * ctx->n_context + pos0) * ctx->kv_dim;
        const size_t hoff = (size_t)l * npos * ctx->kv_dim;
        for (int q = 0; q < 2; q++) {
            uint16_t* dev = (q ? ctx->vc : ctx->kc) + doff;
            uint16_t* host = (q ? vh : kh);
            if (!host) continue;
            const hipError_t e = write ? hipMemcpyAsync(dev, host + hoff, row * npos, hipMemcpyHostToDevice, ctx->stream)
                                       : hipMemcpyAsync(host + hoff, dev, row * npos, hipMemcpyDeviceToHost, ctx->stream);
            if (e != hipSuccess) { lg_set_error("kv copy: %s", hipGetErrorString(e)); return ctx_fail(ctx, LG_ERR_HIP); }
        }
    }
    return lg_sync(ctx);
}

extern "C" int lg_kv_read(lg_ctx* ctx, int layer0, int nlayers, int pos0, int npos, uint16_t* k_host, uint16_t* v_host)
{
    return kv_io(ctx, layer0, nlayers, pos0, npos, k_host, v_host, false);
}

extern "C" int lg_kv_write(lg_ctx* ctx, int layer0, int nlayers, int pos0, int npos, const uint16_t* k_host,
                           const uint16_t* v_host)
{
    return kv_io(ctx, layer0, nlayers, pos0, npos, (uint16_t*)k_host, (uint16_t*)v_host, true);
}

/* ------------------------------------------------------------------ */
/* state files (save_model_state / load_model_state,                   */
/* fast/ligguf_fast_qk.cpp:216-302)                                     */
/* ------------------------------------------------------------------ */
/* model_file (fast/common.h:26-31): packed, little-endian */
#pragma pack(push, 1)
struct lg_model_file {
    int32_t pos;
    int32_t n_context;
    uint64_t kv_size;       /* n_layers * pos * kv_dim fp16 values per cache */
    uint64_t logits_size;   /* vocab floats */
};
#pragma pack(pop)
static_assert(sizeof(lg_model_file) == 24, "model_file is 24 packed bytes");

/* pinned staging for one layer's K or V block or the logits */
struct lg_pinned {
    void* p = nullptr;
    ~lg_pinned() { if (p) hipHostFree(p); }
};

extern "C" int lg_state_save(lg_ctx* ctx, const char* path, int pos)
{
    if (!ctx || !path) { lg_set_error("lg_state_save: null argument"); return ctx_fail(ctx, LG_ERR_ARG); }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    /* the reference refuses an empty state (fast/ligguf_fast_qk.cpp:266-269) */
    if (pos <= 0 || pos > ctx->n_context) {
        lg_set_error("lg_state_save: position %d outside 1..%d", pos, ctx->n_context);
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    hipSetDevice(ctx->device);
    LG_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    const size_t blk = (size_t)pos * ctx->kv_dim * 2, lbytes = (size_t)ctx->vocab * 4;
    lg_pinned buf;
    LG_HIP_CHECK(hipHostMalloc(&buf.p, std::max(blk, lbytes), 0));
    FILE* f = fopen(path, "wb");
    if (!f) { lg_set_error("lg_state_save: cannot create %s", path); return ctx_fail(ctx, LG_ERR_ARG); }
    lg_model_file hdr = {};
    hdr.pos = pos;
    hdr.n_context = ctx->n_context;
    hdr.kv_size = (uint64_t)ctx->n_layers * pos * ctx->kv_dim;
    hdr.logits_size = (uint64_t)ctx->vocab;
    bool ok = fwrite(&hdr, sizeof(hdr), 1, f) == 1;
    for (int q = 0; q < 2 && ok; q++) {
        const uint16_t* cache = q ? ctx->vc : ctx->kc;
        for (int l = 0; l < ctx->n_layers && ok; l++) {
            const hipError_t e = hipMemcpy(buf.p, cache + (size_t)l * ctx->n_context * ctx->kv_dim, blk,
                                           hipMemcpyDeviceToHost);
            ok = e == hipSuccess && fwrite(buf.p, blk, 1, f) == 1;
        }
    }
    if (ok) ok = hipMemcpy(buf.p, ctx->logits, lbytes, hipMemcpyDeviceToHost) == hipSuccess &&
                 fwrite(buf.p, lbytes, 1, f) == 1;
    if (fclose(f) != 0) ok = false;
    if (!ok) { lg_set_error("lg_state_save: writing %s failed", path); return ctx_fail(ctx, LG_ERR_STATE); }
    return LG_OK;
}

extern "C" int lg_state_load(lg_ctx* ctx, const char* path, int* pos_out, float* logits_host)
{
    if (!ctx || !path) { lg_set_error("lg_state_load: null argument"); return ctx_fail(ctx, LG_ERR_ARG); }
    if (!ctx->loaded) { lg_set_error("no model loaded"); return ctx_fail(ctx, LG_ERR_STATE); }
    hipSetDevice(ctx->device);
    FILE* f = fopen(path, "rb");
    if (!f) { lg_set_error("lg_state_load: cannot read %s", path); return ctx_fail(ctx, LG_ERR_ARG); }
    lg_model_file hdr = {};
    /* the checks of load_model_state (fast/ligguf_fast_qk.cpp:229-235,250) */
    bool ok = fread(&hdr, sizeof(hdr), 1, f) == 1 && hdr.kv_size && hdr.logits_size && hdr.pos > 0 &&
              hdr.pos <= ctx->n_context && hdr.kv_size == (uint64_t)ctx->n_layers * hdr.pos * ctx->kv_dim &&
              hdr.logits_size == (uint64_t)ctx->vocab;
    if (!ok) {
        fclose(f);
        lg_set_error("lg_state_load: %s is not a state file of this model (pos %d, kv %llu, logits %llu)", path,
                     hdr.pos, (unsigned long long)hdr.kv_size, (unsigned long long)hdr.logits_size);
        return ctx_fail(ctx, LG_ERR_ARG);
    }
    const int pos = hdr.pos;
    const size_t blk = (size_t)pos * ctx->kv_dim * 2, lbytes = (size_t)ctx->vocab * 4;
    /* load_model_state reads into a copy and keeps the old state when a
     * read fails (fast/ligguf_fast_qk.cpp:224-259); here the file must hold
     * every block before the first one reaches the cache, so a short file
     * leaves the cache untouched */
    const uint64_t need = sizeof(hdr) + 2 * hdr.kv_size * 2 + hdr.logits_size * 4;
    struct stat fst;
    if (fstat(fileno(f), &fst) || (uint64_t)fst.st_size < need) {
        fclose(f);
        lg_set_error("lg_state_load: %s is truncated (%lld bytes, %llu needed)", path, (long long)fst.st_size,
                     (unsigned long long)need);
        return ctx_fail(ctx, LG_ERR_STATE);
    }
    lg_pinned buf;
    const hipError_t ea = hipHostMalloc(&buf.p, std::max(blk, lbytes), 0);
    if (ea != hipSuccess) {
        fclose(f);
        lg_set_error("lg_state_load: pinned staging: %s", hipGetErrorString(ea));
        return ctx_fail(ctx, LG_ERR_NOMEM);
    }
    LG_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    for (int q = 0; q < 2 && ok; q++) {
        uint16_t* cache = q ? ctx->vc : ctx->kc;
        for (int l = 0; l < ctx->n_layers && ok; l++)
            ok = fread(buf.p, blk, 1, f) == 1 &&
                 hipMemcpy(cache + (size_t)l * ctx->n_context * ctx->kv_dim, buf.p, blk, hipMemcpyHostToDevice) ==
                     hipSuccess;
    }
    if (ok) ok = fread(buf.p, lbytes, 1, f) == 1 &&
                 hipMemcpy(ctx->logits, buf.p, lbytes, hipMemcpyHostToDevice) == hipSuccess;
    fclose(f);
    if (!ok) { lg_set_error("lg_state_load: reading %s failed", path); return ctx_fail(ctx, LG_ERR_STATE); }
    if (logits_host) memcpy(logits_host, buf.p, lbytes);
    /* the device step record and the last greedy token no longer describe the state */
    ctx->dev_known = false;
    ctx->last_was_pk = false;
    if (pos_out) *pos_out = pos;
    return LG_OK;
}

/* ------------------------------------------------------------------ */
/* per-op entry points                                                  */
/* ------------------------------------------------------------------ */
#define S(stream) ((hipStream_t)(stream))

extern "C" int lg_dequantize_row(int type, const void* x, float* y, int64_t n, void* stream)
{
    return lg_launch_dequantize(type, x, y, n, S(stream));
}

extern "C" int lg_quantize_q8_0(const float* x, int64_t n, void* y, void* stream)
{
    return lg_launch_quantize_q8_0(x, n, y, S(stream));
}

extern "C" int lg_quantize_q8_K(const float* x, int64_t n, void* y, void* stream)
{
    return lg_launch_quantize_q8_K(x, n, y, S(stream));
}

extern "C" int lg_matvec(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, int accumulate,
                         void* stream)
{
    return lg_launch_matvec(type, w, rsz, n, d, xq, out, accumulate, S(stream));
}

extern "C" int lg_rmsnorm_quant(const float* x, const float* w, int n, float eps, int qtype, void* out_q, float* out_f,
                                void* stream)
{
    return lg_launch_rmsnorm_quant(x, w, n, eps, qtype, out_q, out_f, S(stream));
}

extern "C" int lg_qk_norm_rope_kv(float* q, float* k, const float* v, const float* qw, const float* kw, int n_heads,
                                  int n_kv_heads, int head_dim, int rope_dim, int pos, const float* freq, float eps,
                                  uint16_t* kc_row, uint16_t* vc_row, void* stream)
{
    return lg_launch_qk_norm_rope_kv(q, k, v, qw, kw, n_heads, n_kv_heads, head_dim, rope_dim, pos, freq, eps, kc_row,
                                     vc_row, S(stream));
}

extern "C" size_t lg_attn_workspace_size(int n_heads, int head_dim, int pos)
{
    return lg_attn_ws_bytes(n_heads, head_dim, pos);
}

extern "C" int lg_attn_decode(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                              int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* workspace,
                              size_t workspace_bytes, void* stream)
{
    return lg_launch_attn(q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos, out, workspace, workspace_bytes,
                          S(stream));
}

extern "C" int lg_swiglu_quant(float* hb, const float* hb2, int n, int qtype, void* out_q, void* stream)
{
    return lg_launch_swiglu_quant(hb, hb2, n, qtype, out_q, S(stream));
}
