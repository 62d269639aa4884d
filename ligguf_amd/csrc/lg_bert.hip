/* lg_bert.hip -- BERT sentence embedding (bert_embed, fast/vdb.cpp:123-245)
 * and the vector-memory search (vdb_query, fast/vdb.cpp:337-377) on gfx950.
 *
 * A pass runs T tokens -- one sequence or several, each attending only to
 * itself -- through the encoder:
 *   embedding sum + LayerNorm -> per layer { Q|K|V GEMM (+bias) ->
 *   bidirectional attention per sequence and head -> att_out GEMM (+bias
 *   +residual) -> LayerNorm -> up GEMM (+bias, GELU) -> down GEMM (+bias
 *   +residual) -> LayerNorm } -> mean over each sequence + L2 norm.
 * The reference runs the same arithmetic a token at a time through
 * matmul3/matmul (fast/lil_math.cpp:748-899); here each weight matrix is read
 * once per pass and multiplied on MFMA:
 *   - F32/F16 matrices x fp32 activations on v_mfma_f32_16x16x4f32: the
 *     products of dot_f32 / dot_f16_f32 exactly, fp32 accumulation;
 *   - Q8_0/Q1_0/Q1_G matrices, repacked at upload into int8 values (the
 *     Q8_0 quants, or +-1 from the sign bits) and one fp32 scale per 32 --
 *     x Q8_0 activations (quantize_q8_0 per token, the same lane quantizer
 *     as the decode step) on v_mfma_i32_16x16x32_i8: the integer block sums
 *     of dot_q8_0_q8_0 / _q1_0 / _q1_G (fast/lil_math.cpp:411-462) exactly,
 *     then scale_w * scale_a * sum accumulated block by block in fp32.
 * LayerNorm takes mean and variance in double, as the reference's layernorm
 * (fast/lil_math.cpp:948-962) does; attention, GELU, pooling and the L2 norm
 * are fp32 as in the reference (:939-984, fast/vdb.cpp:189-244).  Only the
 * fp32 summation orders differ from the reference.
 *
 * HBM layout: the encoder's matrices (F32/F16 rows as stored, int8 [rows]
 * [cols] + scales [cols/32][rows] otherwise; Q|K|V stacked into one matrix
 * when their forms agree), fp32 activations [T][width] per buffer, the Q8_0
 * activation of the next GEMM as int8 [T][width] + scales [width/32][T],
 * and the vector memory as fp16 rows [n][n_embed].
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <vector>

#include "lg_common.h"
#include "lg_prefill.h"
#include "lg_quant.h"

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

/* matrix forms on the device: LG_F32 / LG_F16 as stored, or BF_I8 */
#define BF_I8 100
#define BERT_HD_MAX 128
#define BERT_NCTX_MAX 4096
#define BERT_NE_MAX 4096
#define BERT_SP 16384          /* LDS floats for one attention block's scores */
#define LG_VDB_KMAX 8
#define VDB_BLOCKS_MAX 1024

/* ------------------------------------------------------------------ */
/* device helpers                                                       */
/* ------------------------------------------------------------------ */
__device__ __forceinline__ double b_block_sum_d(double v, double* red)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();                     /* red is reused by consecutive sums */
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

/* Q8_0 of the wave's 256 values (chunk c of the row): lane l holds values
 * 256c + 4l .. +3 (zeros past n); quants to qrow, the fp16-rounded block
 * scales to qd[block][t] (tokens contiguous) */
__device__ __forceinline__ void b_emit_q8(const float v[4], int8_t* __restrict__ qrow, float* __restrict__ qd, int ldd,
                                          int t, int c, int n)
{
    const Q80Lane r = lg_q8_0_lane(v);
    const int lane = threadIdx.x & 63;
    const int i0 = 256 * c + 4 * lane;
    if (i0 < n) {
        *(uint32_t*)(qrow + i0) = r.packed;
        if ((lane & 7) == 0) qd[(size_t)(i0 >> 5) * ldd + t] = lg_h2f(lg_f2h(r.d));
    }
}

/* layernorm (fast/lil_math.cpp:948-962) of one row held by a 256-thread
 * block: thread (wave w, lane l) holds values 1024p + 256w + 4l .. +3.
 * mean and variance in double, scale = 1/sqrtf(var + eps) in float, the
 * output (x - mean) * scale * w + b in double rounded to float. */
template <int NP>
__device__ __forceinline__ void b_layernorm(float (&v)[NP][4], int n, const float* __restrict__ w,
                                            const float* __restrict__ bias, float eps, double* red,
                                            float* __restrict__ out, int8_t* __restrict__ q, float* __restrict__ qd,
                                            int ldd, int t)
{
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    double s = 0.0;
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (1024 * p + 256 * wv + 4 * lane + j < n) s += (double)v[p][j];
    const double mean = b_block_sum_d(s, red) / n;
    double s2 = 0.0;
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (1024 * p + 256 * wv + 4 * lane + j < n) {
                const double dd = (double)v[p][j] - mean;
                s2 += dd * dd;
            }
    const double var = b_block_sum_d(s2, red) / n;
    const float scale = 1.0f / sqrtf((float)(var + (double)eps));
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = 1024 * p + 256 * wv + 4 * lane;
        if (1024 * p + 256 * wv >= n) break;        /* wave-uniform */
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            o[j] = i0 + j < n ? (float)(((double)v[p][j] - mean) * (double)scale * (double)w[i0 + j] + (double)bias[i0 + j])
                              : 0.0f;
        if (i0 < n) *(float4*)(out + i0) = make_float4(o[0], o[1], o[2], o[3]);
        if (q) b_emit_q8(o, q, qd, ldd, t, 4 * p + wv, n);
    }
}

/* ------------------------------------------------------------------ */
/* embeddings + LayerNorm (fast/vdb.cpp:155-168)                        */
/* ------------------------------------------------------------------ */
struct BEmbArgs {
    const uint8_t *tok, *pos, *typ;
    int tok_t, pos_t, typ_t;
    uint32_t tok_rsz, pos_rsz;
    const int2* tokpos;        /* [T] {token id, position in its sequence} */
    const float *w, *b;
    float eps;
    int n;
    float* out;
    int8_t* q;                 /* optional Q8_0 of the output */
    float* qd;
    int ldd;
};

template <int NP>
__global__ __launch_bounds__(256) void k_bert_embed(BEmbArgs a)
{
    __shared__ double red[4];
    const int t = blockIdx.x;
    const int2 tp = a.tokpos[t];
    const uint8_t* tr = a.tok + (size_t)tp.x * a.tok_rsz;
    const uint8_t* pr = a.pos + (size_t)tp.y * a.pos_rsz;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    float v[NP][4];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = 1024 * p + 256 * wv + 4 * lane + j;
            v[p][j] = i < a.n ? (lg_dq_value(a.tok_t, tr, i) + lg_dq_value(a.pos_t, pr, i)) + lg_dq_value(a.typ_t, a.typ, i)
                              : 0.0f;
        }
    b_layernorm<NP>(v, a.n, a.w, a.b, a.eps, red, a.out + (size_t)t * a.n, a.q ? a.q + (size_t)t * a.n : nullptr, a.qd,
                    a.ldd, t);
}

/* LayerNorm of row t of y (n wide) into out, optionally quantized */
template <int NP>
__global__ __launch_bounds__(256) void k_bert_ln(const float* __restrict__ y, int n, const float* __restrict__ w,
                                                 const float* __restrict__ b, float eps, float* __restrict__ out,
                                                 int8_t* __restrict__ q, float* __restrict__ qd, int ldd)
{
    __shared__ double red[4];
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const float* row = y + (size_t)t * n;
    float v[NP][4];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = 1024 * p + 256 * wv + 4 * lane;
        const float4 x = i0 < n ? *(const float4*)(row + i0) : make_float4(0.f, 0.f, 0.f, 0.f);
        v[p][0] = x.x; v[p][1] = x.y; v[p][2] = x.z; v[p][3] = x.w;
    }
    b_layernorm<NP>(v, n, w, b, eps, red, out + (size_t)t * n, q ? q + (size_t)t * n : nullptr, qd, ldd, t);
}

/* Q8_0 of row t of x (n wide): the quantize_q8_0 matmul() applies before a
 * Q8_0/Q1 product (fast/lil_math.cpp:751-755) */
__global__ __launch_bounds__(256) void k_bert_quant(const float* __restrict__ x, int n, int8_t* __restrict__ q,
                                                    float* __restrict__ qd, int ldd)
{
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const float* row = x + (size_t)t * n;
    for (int c = wv; 256 * c < n; c += 4) {
        const int i0 = 256 * c + 4 * lane;
        const float4 f = i0 < n ? *(const float4*)(row + i0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float v[4] = {f.x, f.y, f.z, f.w};
        b_emit_q8(v, q + (size_t)t * n, qd, ldd, t, c, n);
    }
}

/* ------------------------------------------------------------------ */
/* token-batched GEMM: out[t][r] = W[r] . act[t] (+ epilogue)           */
/* ------------------------------------------------------------------ */
enum { EP_BIAS = 0, EP_BIAS_RES = 1, EP_BIAS_GELU = 2, EP_STORE = 3, EP_ADD = 4 };   /* STORE/ADD: no bias; ADD: out += */

struct BGemm {
    const uint8_t* w;          /* F32/F16: [R][K]; BF_I8: int8 [R][K] */
    const float* wd;           /* BF_I8: [K/32][R] */
    int R, K;
    const float* x;            /* fp32 activations [T][ldx] (F32/F16) */
    int ldx;
    const int8_t* q;           /* Q8_0 activations [T][K] (BF_I8) */
    const float* qd;           /* [K/32][ldd] */
    int ldd;
    int T;
    const float* bias;         /* [R] */
    const float* res;          /* [T][ldr] residual (EP_BIAS_RES) */
    int ldr;
    float* out;                /* [T][ldo] */
    int ldo;
};

/* One wave per (16 TM)-token x (16 TN)-row tile (TM x TN MFMA tiles of
 * 16 x 16; the launcher picks the largest tile that still gives the grid
 * enough waves).  MFMA operand A holds tokens (M), B weight rows (N); the
 * output D[m][n] of a 16 x 16 tile sits in lane (g = l/16, m = l%16) as
 * tokens 4g..4g+3, row m.  fp32 form: per 32-value chunk, lane group g
 * takes values 8g..8g+7 of its token and its row, and MFMA step j (of 8)
 * multiplies value 8g+j -- the four lane groups give the K = 4 of each
 * step, so the eight steps cover the chunk.  int8 form: one
 * v_mfma_i32_16x16x32_i8 per 32-value block (lane group g: bytes
 * 8g..8g+7), the block's integer sum scaled by both block scales. */
template <int WT, int EP, int TM, int TN>
__global__ __launch_bounds__(64) void k_bert_gemm(BGemm a)
{
    const int lane = threadIdx.x, g = lane >> 4, m = lane & 15;
    const int ntt = (a.T + 16 * TM - 1) / (16 * TM);
    const int t0 = (blockIdx.x % ntt) * 16 * TM, r0 = (blockIdx.x / ntt) * 16 * TN;
    int tr[TM], wr[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) tr[i] = min(t0 + 16 * i + m, a.T - 1);
#pragma unroll
    for (int j = 0; j < TN; j++) wr[j] = min(r0 + 16 * j + m, a.R - 1);
    v4f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    /* NPF chunks of 32 values in flight: chunk c sits in register slot
     * c % NPF, loaded NPF - 1 chunks before it is multiplied */
    constexpr int NPF = 4;
    if constexpr (WT == BF_I8) {
        const int8_t* ap[TM];
        const int8_t* bp[TN];
#pragma unroll
        for (int i = 0; i < TM; i++) ap[i] = a.q + (size_t)tr[i] * a.K + 8 * g;
#pragma unroll
        for (int j = 0; j < TN; j++) bp[j] = (const int8_t*)a.w + (size_t)wr[j] * a.K + 8 * g;
        const int nb = a.K >> 5;
        long av[NPF][TM], bv[NPF][TN];
        float4 xd[NPF][TM];
        float wdv[NPF][TN];
        auto load = [&](int u, int b) {
#pragma unroll
            for (int i = 0; i < TM; i++) {
                av[u][i] = *(const long*)(ap[i] + 32 * b);
                xd[u][i] = *(const float4*)(a.qd + (size_t)b * a.ldd + t0 + 16 * i + 4 * g);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                bv[u][j] = *(const long*)(bp[j] + 32 * b);
                wdv[u][j] = a.wd[(size_t)b * a.R + wr[j]];
            }
        };
#pragma unroll
        for (int u = 0; u < NPF - 1; u++)
            if (u < nb) load(u, u);
        for (int b0 = 0; b0 < nb; b0 += NPF) {
#pragma unroll
            for (int u = 0; u < NPF; u++) {
                const int b = b0 + u;
                if (b + NPF - 1 < nb) load((u + NPF - 1) % NPF, b + NPF - 1);
                if (b < nb) {
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const float xs[4] = {xd[u][i].x, xd[u][i].y, xd[u][i].z, xd[u][i].w};
#pragma unroll
                        for (int j = 0; j < TN; j++) {
                            const v4i sm = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][i], bv[u][j], (v4i){0, 0, 0, 0},
                                                                                 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                acc[i][j][v] = __builtin_fmaf(xs[v] * wdv[u][j], (float)sm[v], acc[i][j][v]);
                        }
                    }
                }
            }
        }
    } else {
        constexpr int ESZ = WT == LG_F32 ? 4 : 2;
        const float* ap[TM];
        const uint8_t* bp[TN];
#pragma unroll
        for (int i = 0; i < TM; i++) ap[i] = a.x + (size_t)tr[i] * a.ldx + 8 * g;
#pragma unroll
        for (int j = 0; j < TN; j++) bp[j] = a.w + ((size_t)wr[j] * a.K + 8 * g) * ESZ;
        float4 A[NPF][TM][2];
        uint4 B[NPF][TN][ESZ / 2];
        auto load = [&](int u, int k0) {
#pragma unroll
            for (int i = 0; i < TM; i++) {
                A[u][i][0] = *(const float4*)(ap[i] + k0);
                A[u][i][1] = *(const float4*)(ap[i] + k0 + 4);
            }
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int h = 0; h < ESZ / 2; h++) B[u][j][h] = *(const uint4*)(bp[j] + (size_t)k0 * ESZ + 16 * h);
        };
        const int nc = a.K >> 5;
#pragma unroll
        for (int u = 0; u < NPF - 1; u++)
            if (u < nc) load(u, 32 * u);
        for (int c0 = 0; c0 < nc; c0 += NPF) {
#pragma unroll
            for (int u = 0; u < NPF; u++) {
                const int c = c0 + u;
                if (c + NPF - 1 < nc) load((u + NPF - 1) % NPF, 32 * (c + NPF - 1));
                if (c < nc) {
                    float af[TM][8], bf[TN][8];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        af[i][0] = A[u][i][0].x; af[i][1] = A[u][i][0].y; af[i][2] = A[u][i][0].z; af[i][3] = A[u][i][0].w;
                        af[i][4] = A[u][i][1].x; af[i][5] = A[u][i][1].y; af[i][6] = A[u][i][1].z; af[i][7] = A[u][i][1].w;
                    }
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        if constexpr (WT == LG_F32) {
#pragma unroll
                            for (int h = 0; h < 2; h++) {
                                bf[j][4 * h + 0] = __uint_as_float(B[u][j][h].x);
                                bf[j][4 * h + 1] = __uint_as_float(B[u][j][h].y);
                                bf[j][4 * h + 2] = __uint_as_float(B[u][j][h].z);
                                bf[j][4 * h + 3] = __uint_as_float(B[u][j][h].w);
                            }
                        } else {
                            const uint32_t uu[4] = {B[u][j][0].x, B[u][j][0].y, B[u][j][0].z, B[u][j][0].w};
#pragma unroll
                            for (int h = 0; h < 4; h++) {
                                bf[j][2 * h] = lg_h2f((uint16_t)(uu[h] & 0xffffu));
                                bf[j][2 * h + 1] = lg_h2f((uint16_t)(uu[h] >> 16));
                            }
                        }
                    }
#pragma unroll
                    for (int st = 0; st < 8; st++)
#pragma unroll
                        for (int i = 0; i < TM; i++)
#pragma unroll
                            for (int j = 0; j < TN; j++)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][st], bf[j][st], acc[i][j], 0, 0, 0);
                }
            }
        }
    }

#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int r = r0 + 16 * j + m;
        if (r >= a.R) continue;
        const float bias = EP <= EP_BIAS_GELU ? a.bias[r] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = t0 + 16 * i + 4 * g + v;
                if (t >= a.T) continue;
                float o = acc[i][j][v];
                if constexpr (EP == EP_STORE) {
                } else if constexpr (EP == EP_ADD) {
                    o = a.out[(size_t)t * a.ldo + r] + o;
                } else if constexpr (EP == EP_BIAS) {
                    o = o + bias;
                } else if constexpr (EP == EP_BIAS_RES) {
                    o = o + (bias + a.res[(size_t)t * a.ldr + r]);
                } else {
                    /* gelu (fast/lil_math.cpp:978-984) of row + bias */
                    const float u = o + bias;
                    o = 0.5f * u * (1.0f + tanhf(0.7978845608f * (u + 0.044715f * u * u * u)));
                }
                a.out[(size_t)t * a.ldo + r] = o;
            }
    }
}

/* ------------------------------------------------------------------ */
/* bidirectional attention (fast/vdb.cpp:189-212)                       */
/* ------------------------------------------------------------------ */
/* One block per (block of qb query tokens of one sequence, head).  K and V
 * rows of the head stream through LDS in tiles of 64 positions; the qb
 * score rows (the whole sequence) stay in LDS: scores = q.k * scale, then
 * the reference's softmax (max, expf, sum, divide), then ctx = sum_t p_t v_t
 * in position order.  tpr = 256/qb threads share a query row. */
struct BAttnBlk {
    int q0, nq, s0, n;         /* first query token, queries, sequence start and length */
};

template <int HD>
__global__ __launch_bounds__(256) void k_bert_attn(const float* __restrict__ qkv, int ne,
                                                   const BAttnBlk* __restrict__ blks, int qb, int pst, float scale,
                                                   float* __restrict__ ctx)
{
    __shared__ float s_p[BERT_SP];
    __shared__ float s_q[16][HD];
    __shared__ float s_kv[64][HD + 1];
    const BAttnBlk bk = blks[blockIdx.x];
    const int h = blockIdx.y, tid = threadIdx.x;
    const int tpr = 256 / qb;
    const int qi = tid / tpr, kk = tid % tpr;
    const size_t ld = 3 * (size_t)ne;
    float* prow = s_p + qi * pst;

    for (int idx = tid; idx < qb * HD; idx += 256) {
        const int r = idx / HD, d = idx % HD;
        s_q[r][d] = qkv[(size_t)(bk.q0 + min(r, bk.nq - 1)) * ld + h * HD + d];
    }
    for (int kt = 0; kt < bk.n; kt += 64) {
        __syncthreads();
        for (int idx = tid; idx < 64 * HD; idx += 256) {
            const int r = idx / HD, d = idx % HD;
            s_kv[r][d] = kt + r < bk.n ? qkv[(size_t)(bk.s0 + kt + r) * ld + ne + h * HD + d] : 0.0f;
        }
        __syncthreads();
        for (int kj = kk; kj < 64; kj += tpr) {
            float acc = 0.0f;
#pragma unroll 16
            for (int d = 0; d < HD; d++) acc = __builtin_fmaf(s_q[qi][d], s_kv[kj][d], acc);
            if (kt + kj < bk.n) prow[kt + kj] = acc * scale;
        }
    }
    __syncthreads();
    /* softmax (fast/lil_math.cpp:964-976) over the row, tpr lanes per row */
    float mx = -INFINITY;
    for (int c = kk; c < bk.n; c += tpr) mx = fmaxf(mx, prow[c]);
    for (int o = tpr >> 1; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.0f;
    for (int c = kk; c < bk.n; c += tpr) {
        const float e = expf(prow[c] - mx);
        prow[c] = e;
        sum += e;
    }
    for (int o = tpr >> 1; o; o >>= 1) sum += __shfl_xor(sum, o);
    for (int c = kk; c < bk.n; c += tpr) prow[c] = prow[c] / sum;

    constexpr int DPT = HD / 16;
    float acc[DPT];
#pragma unroll
    for (int u = 0; u < DPT; u++) acc[u] = 0.0f;
    for (int kt = 0; kt < bk.n; kt += 64) {
        __syncthreads();
        for (int idx = tid; idx < 64 * HD; idx += 256) {
            const int r = idx / HD, d = idx % HD;
            s_kv[r][d] = kt + r < bk.n ? qkv[(size_t)(bk.s0 + kt + r) * ld + 2 * ne + h * HD + d] : 0.0f;
        }
        __syncthreads();
        const int kn = min(64, bk.n - kt);
        for (int kj = 0; kj < kn; kj++) {
            const float p = prow[kt + kj];
#pragma unroll
            for (int u = 0; u < DPT; u++) {
                const int d = kk + tpr * u;
                if (d < HD) acc[u] = __builtin_fmaf(p, s_kv[kj][d], acc[u]);
            }
        }
    }
    if (qi < bk.nq) {
#pragma unroll
        for (int u = 0; u < DPT; u++) {
            const int d = kk + tpr * u;
            if (d < HD) ctx[(size_t)(bk.q0 + qi) * ne + h * HD + d] = acc[u];
        }
    }
}

/* The same on fp32 MFMA for sequences of up to PMAX positions: one block
 * per (16 query tokens of one sequence, head), 4 waves.  K, then V, come
 * into LDS in chunks of KC positions, each chunk with all its loads in
 * flight at once (the sequence is short: a handful of round trips in all).
 * Scores: wave w takes the 16-key tiles 16w, 16w+64, ... of a chunk; a
 * tile is S[q][key] = sum_d Q[q][d] K[key][d], HD/4 v_mfma_f32_16x16x4f32
 * (A = Q: lane (g, m) holds Q[m][d0+g]; B = K^T: K[key0+m][d0+g]; D:
 * queries 4g..4g+3, key m), scaled and kept in LDS.  The reference's
 * softmax runs on the rows as in k_bert_attn.  Then O[q][d] = sum_key
 * P[q][key] V[key][d]: per 4 keys one MFMA per 16 dims (A = P:
 * P[m][key0+g]; B = V: V[key0+g][16 dt + m]), wave w over the w-th quarter
 * of each chunk; the four waves' partial O are summed in LDS.  LDS rows are
 * padded to an odd number of floats so the 16 rows a lane group reads fall
 * in distinct banks. */
template <int HD, int PMAX>
struct BAttnChunk {
    static constexpr int KC0 = HD <= 64 ? 256 : 128;
    static constexpr int KC = KC0 < PMAX ? KC0 : PMAX;   /* positions per K/V chunk */
};

template <int HD, int PMAX>
__global__ __launch_bounds__(256) void k_bert_attn_mfma(const float* __restrict__ qkv, int ne,
                                                        const BAttnBlk* __restrict__ blks, float scale,
                                                        float* __restrict__ ctx)
{
    constexpr int LD = HD + 1, PS = PMAX + 1, NDT = HD / 16, KC = BAttnChunk<HD, PMAX>::KC, H4 = HD / 4;
    __shared__ float s_q[16 * LD];
    __shared__ float s_kv[KC * LD];
    __shared__ float s_p[16 * PS];
    const BAttnBlk bk = blks[blockIdx.x];
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, m = lane & 15;
    const size_t ld = 3 * (size_t)ne;

    /* rows [c0, c0 + KC) of the head's K (off = ne) or V (off = 2 ne) into s_kv */
    auto load_chunk = [&](int c0, int off) {
        for (int idx = tid; idx < KC * H4; idx += 256) {
            const int r = idx / H4, c4 = idx % H4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c0 + r < bk.n) v = *(const float4*)(qkv + (size_t)(bk.s0 + c0 + r) * ld + off + h * HD + 4 * c4);
            float* d = s_kv + r * LD + 4 * c4;
            d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
        }
    };

    for (int idx = tid; idx < 16 * HD; idx += 256) {
        const int r = idx / HD, d = idx % HD;
        s_q[r * LD + d] = qkv[(size_t)(bk.q0 + min(r, bk.nq - 1)) * ld + h * HD + d];
    }
    for (int c0 = 0; c0 < bk.n; c0 += KC) {
        __syncthreads();
        load_chunk(c0, ne);
        __syncthreads();
        const int kn = min(KC, bk.n - c0);
        for (int k16 = 16 * w; k16 < kn; k16 += 64) {
            v4f acc = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d0 = 0; d0 < HD; d0 += 4)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s_q[m * LD + d0 + g], s_kv[(k16 + m) * LD + d0 + g], acc, 0, 0,
                                                           0);
            const int key = c0 + k16 + m;
            if (key < bk.n) {
#pragma unroll
                for (int v = 0; v < 4; v++) s_p[(4 * g + v) * PS + key] = acc[v] * scale;
            }
        }
    }
    __syncthreads();
    {
        /* softmax (fast/lil_math.cpp:964-976), 16 lanes per row */
        const int qi = tid >> 4, kk = tid & 15;
        float* prow = s_p + qi * PS;
        float mx = -INFINITY;
        for (int c = kk; c < bk.n; c += 16) mx = fmaxf(mx, prow[c]);
#pragma unroll
        for (int o = 8; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float sum = 0.0f;
        for (int c = kk; c < bk.n; c += 16) {
            const float e = expf(prow[c] - mx);
            prow[c] = e;
            sum += e;
        }
#pragma unroll
        for (int o = 8; o; o >>= 1) sum += __shfl_xor(sum, o);
        for (int c = kk; c < bk.n; c += 16) prow[c] = prow[c] / sum;
    }
    v4f o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = (v4f){0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < bk.n; c0 += KC) {
        __syncthreads();
        load_chunk(c0, 2 * ne);
        __syncthreads();
        const int kq = min(KC / 4, max(0, bk.n - c0 - w * (KC / 4)));   /* keys of this wave's quarter */
        for (int k4 = 0; k4 < kq; k4 += 4) {
            const int kl = w * (KC / 4) + k4;                            /* chunk-local key of the step */
            const float pa = c0 + kl + g < bk.n ? s_p[m * PS + c0 + kl + g] : 0.0f;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, s_kv[(kl + g) * LD + 16 * dt + m], o[dt], 0, 0, 0);
        }
    }
    __syncthreads();
    float* s_o = s_kv;                                   /* [4 waves][16 queries][HD] */
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) s_o[(w * 16 + 4 * g + v) * HD + 16 * dt + m] = o[dt][v];
    __syncthreads();
    for (int idx = tid; idx < 16 * HD; idx += 256) {
        const int q = idx / HD, d = idx % HD;
        if (q < bk.nq)
            ctx[(size_t)(bk.q0 + q) * ne + h * HD + d] =
                ((s_o[q * HD + d] + s_o[(16 + q) * HD + d]) + s_o[(32 + q) * HD + d]) + s_o[(48 + q) * HD + d];
    }
}

/* ------------------------------------------------------------------ */
/* mean over the sequence + l2norm (fast/vdb.cpp:237-244,              */
/* fast/lil_math.cpp:939-946)                                           */
/* ------------------------------------------------------------------ */
/* sums over the sequence: block (sequence, 64 columns), 1024 threads =
 * 64 columns x 16 position groups; group j adds positions j, j+16, ... and
 * the 16 partial sums are added in order, then divided by the length
 * (out[i] /= ntok) into mean[seq][n] */
__global__ __launch_bounds__(1024) void k_bert_pool_mean(const float* __restrict__ x, int ne,
                                                         const int2* __restrict__ seqs, float* __restrict__ mean)
{
    __shared__ float s_part[16][64];
    const int2 sq = seqs[blockIdx.x];
    const int dg = threadIdx.x & 63, tg = threadIdx.x >> 6;
    const int i = blockIdx.y * 64 + dg;
    float s = 0.0f;
    if (i < ne) {
        const float* base = x + (size_t)sq.x * ne + i;
        int t = tg;
        for (; t + 48 < sq.y; t += 64) {
            const float v0 = base[(size_t)t * ne], v1 = base[(size_t)(t + 16) * ne];
            const float v2 = base[(size_t)(t + 32) * ne], v3 = base[(size_t)(t + 48) * ne];
            s += v0; s += v1; s += v2; s += v3;
        }
        for (; t < sq.y; t += 16) s += base[(size_t)t * ne];
    }
    s_part[tg][dg] = s;
    __syncthreads();
    if (tg == 0 && i < ne) {
        float tot = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) tot += s_part[j][dg];
        mean[(size_t)blockIdx.x * ne + i] = tot / (float)sq.y;
    }
}

/* l2norm (fast/lil_math.cpp:939-946) of each sequence's mean, in place */
__global__ __launch_bounds__(256) void k_bert_l2norm(float* __restrict__ emb, int ne)
{
    __shared__ float red[4];
    float* e = emb + (size_t)blockIdx.x * ne;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < ne; i += 256) ss = __builtin_fmaf(e[i], e[i], ss);
    ss = lg_block_sum(ss, red);
    if (ss <= 0.0f) return;
    const float inv = 1.0f / sqrtf(ss);
    for (int i = threadIdx.x; i < ne; i += 256) e[i] = e[i] * inv;
}

/* ------------------------------------------------------------------ */
/* int8 repack of Q8_0 / Q1_0 / Q1_G rows                               */
/* ------------------------------------------------------------------ */
/* one thread per (row, 32-value block): the block's 32 values as int8
 * (Q8_0 quants; +1 / -1 for set / clear sign bits) and its scale */
__global__ __launch_bounds__(256) void k_bert_repack(int type, const uint8_t* __restrict__ src, uint32_t rsz, int rows,
                                                     int cols, int8_t* __restrict__ q, float* __restrict__ d,
                                                     int r_total, int row_off)
{
    const int nb = cols >> 5;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)rows * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx % nb);
    const uint8_t* row = src + (size_t)r * rsz;
    int8_t* qo = q + (size_t)(row_off + r) * cols + 32 * b;
    float dv = 0.0f;
    if (type == LG_Q8_0) {
        const uint8_t* blk = row + (size_t)b * LG_BS_Q8_0;
        dv = lg_h2f(lg_ld16(blk));
        for (int j = 0; j < 32; j++) qo[j] = (int8_t)blk[2 + j];
    } else if (type == LG_Q1_0) {
        const uint8_t* blk = row + (size_t)b * LG_BS_Q1_0;
        dv = lg_h2f(lg_ld16(blk));
        for (int j = 0; j < 32; j++) qo[j] = ((blk[2 + (j >> 3)] >> (j & 7)) & 1) ? 1 : -1;
    } else {
        const uint8_t* blk = row + (size_t)(b >> 2) * LG_BS_Q1_G;
        dv = lg_h2f(lg_ld16(blk));
        for (int j = 0; j < 32; j++) {
            const int bit = 32 * (b & 3) + j;
            qo[j] = ((blk[2 + (bit >> 3)] >> (bit & 7)) & 1) ? 1 : -1;
        }
    }
    d[(size_t)b * r_total + row_off + r] = dv;
}

/* ------------------------------------------------------------------ */
/* vector memory search (fast/vdb.cpp:352-368)                          */
/* ------------------------------------------------------------------ */
/* An entry's rank key: similarity (order-preserving bits) above the
 * complemented row index, so the larger key is the higher similarity and,
 * among equal ones, the lower row -- the order the reference's
 * strict-greater insertion leaves.  0 is below every real key. */
__device__ __forceinline__ uint64_t vdb_key(float s, int idx)
{
    uint32_t u = __float_as_uint(s);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ float vdb_key_sim(uint64_t k)
{
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __uint_as_float(u);
}

/* keep the LG_VDB_KMAX largest keys, descending */
__device__ __forceinline__ void vdb_insert(uint64_t (&keys)[LG_VDB_KMAX], uint64_t key)
{
#pragma unroll
    for (int j = LG_VDB_KMAX - 1; j >= 0; j--) {
        if (key > keys[j]) keys[j] = (j > 0 && key > keys[j - 1]) ? keys[j - 1] : key;
    }
}

__device__ __forceinline__ uint64_t vdb_wave_max(uint64_t v)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

/* the k largest keys over the block's lists (k rounds: block maximum, the
 * owning thread drops its head); result in out[0..k) of every thread */
__device__ __forceinline__ void vdb_block_topk(uint64_t (&keys)[LG_VDB_KMAX], int k, uint64_t* s_red, uint64_t* out)
{
    for (int r = 0; r < k; r++) {
        const uint64_t wm = vdb_wave_max(keys[0]);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = wm;
        __syncthreads();
        uint64_t best = s_red[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = s_red[w] > best ? s_red[w] : best;
        if (best != 0 && keys[0] == best) {
#pragma unroll
            for (int j = 0; j < LG_VDB_KMAX - 1; j++) keys[j] = keys[j + 1];
            keys[LG_VDB_KMAX - 1] = 0;
        }
        if (threadIdx.x == 0) out[r] = best;
    }
}

/* similarities of the rows: 8 lanes per row, lane s of the group taking
 * values 64c + 8s .. +7; rows at or above the threshold enter the lane's
 * list; the block's k best go to cand[blockIdx.x][k] */
__global__ __launch_bounds__(256) void k_vdb_search(const uint16_t* __restrict__ vecs, int n, int dim,
                                                    const float* __restrict__ emb, float thr, int k,
                                                    uint64_t* __restrict__ cand)
{
    __shared__ float s_e[BERT_NE_MAX];
    __shared__ uint64_t s_red[4];
    __shared__ uint64_t s_out[LG_VDB_KMAX];
    for (int i = threadIdx.x; i < dim; i += 256) s_e[i] = emb[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, grp = lane >> 3, sl = lane & 7;
    uint64_t keys[LG_VDB_KMAX];
#pragma unroll
    for (int j = 0; j < LG_VDB_KMAX; j++) keys[j] = 0;
    const int gw = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nw = (int)((gridDim.x * blockDim.x) >> 6);
    for (int base = gw * 8; base < n; base += nw * 8) {
        const int row = base + grp;
        float acc = 0.0f;
        if (row < n) {
            const uint16_t* rp = vecs + (size_t)row * dim;
            /* each row is read once: nontemporal loads keep it out of the caches */
#pragma unroll 8
            for (int c = 8 * sl; c < dim; c += 64) {
                typedef unsigned int v4u __attribute__((ext_vector_type(4)));
                const v4u hv = __builtin_nontemporal_load((const v4u*)(rp + c));
                const uint32_t u[4] = {hv[0], hv[1], hv[2], hv[3]};
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    acc = __builtin_fmaf(lg_h2f((uint16_t)(u[h] & 0xffffu)), s_e[c + 2 * h], acc);
                    acc = __builtin_fmaf(lg_h2f((uint16_t)(u[h] >> 16)), s_e[c + 2 * h + 1], acc);
                }
            }
        }
        acc = lg_group_sum<8>(acc);
        if (sl == 0 && row < n && acc >= thr) vdb_insert(keys, vdb_key(acc, row));
    }
    vdb_block_topk(keys, k, s_red, s_out);
    __syncthreads();
    if (threadIdx.x < k) cand[(size_t)blockIdx.x * k + threadIdx.x] = s_out[threadIdx.x];
}

/* the k best of nc candidates: out_idx/out_sim and the count found */
__global__ __launch_bounds__(256) void k_vdb_merge(const uint64_t* __restrict__ cand, int nc, int k,
                                                   int* __restrict__ out)
{
    __shared__ uint64_t s_red[4];
    __shared__ uint64_t s_out[LG_VDB_KMAX];
    uint64_t keys[LG_VDB_KMAX];
#pragma unroll
    for (int j = 0; j < LG_VDB_KMAX; j++) keys[j] = 0;
    for (int i = threadIdx.x; i < nc; i += 256) vdb_insert(keys, cand[i]);
    vdb_block_topk(keys, k, s_red, s_out);
    __syncthreads();
    if (threadIdx.x == 0) {
        int cnt = 0;
        for (int r = 0; r < k; r++) {
            const uint64_t key = s_out[r];
            if (key == 0) break;
            out[1 + r] = (int)(0xFFFFFFFFu - (uint32_t)key);
            out[1 + LG_VDB_KMAX + r] = __float_as_int(vdb_key_sim(key));
            cnt++;
        }
        out[0] = cnt;
    }
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */
struct BMat {
    int type = -1;             /* LG_F32, LG_F16 or BF_I8 */
    int rows = 0, cols = 0;
    uint8_t* w = nullptr;
    float* d = nullptr;
};

struct BLayer {
    BMat qkv[3];               /* one stacked matrix (nqkv 1) or q, k, v */
    int nqkv = 1;
    float* qkv_bias = nullptr; /* [3 n_embed] */
    BMat ao, up, down;
    float *ao_bias = nullptr, *up_bias = nullptr, *down_bias = nullptr;
    float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
};

struct lg_bert {
    int device = 0;
    hipStream_t stream = nullptr;
    char err[1024] = {0};
    std::vector<void*> allocs;
    bool loaded = false;
    int n_layers = 0, ne = 0, nh = 0, hd = 0, nff = 0, nctx = 0, vocab = 0, tok_cls = 0, tok_sep = 0;
    float eps = 0.0f;
    int tmax = 0;              /* tokens per pass */
    int tok_t = 0, pos_t = 0, typ_t = 0;
    uint32_t tok_rsz = 0, pos_rsz = 0;
    uint8_t *tok = nullptr, *pos = nullptr, *typ = nullptr;
    float *emb_w = nullptr, *emb_b = nullptr;
    std::vector<BLayer> layers;
    /* activations */
    float *x = nullptr, *x1 = nullptr, *y = nullptr, *qkv = nullptr, *ctx = nullptr, *h = nullptr;
    int8_t* aq = nullptr;
    float* ad = nullptr;
    int ldd = 0;
    /* per-pass tables: tokpos [tmax] int2, attention blocks, sequences */
    void* meta_dev = nullptr;
    uint8_t* meta_host = nullptr;   /* pinned */
    size_t meta_bytes = 0;
    float* emb_dev = nullptr;       /* [tmax/2][ne] pooled embeddings */
    float* emb_host = nullptr;      /* pinned, same size */
    /* vector memory */
    uint16_t* vdb = nullptr;
    int vdb_n = 0, vdb_cap = 0;
    uint64_t* vdb_cand = nullptr;
    int* vdb_out = nullptr;         /* [1 + 2 * KMAX] */
    int* vdb_out_host = nullptr;    /* pinned */
    float* q_emb_dev = nullptr;     /* [ne] query embedding */
    uint8_t* trace = nullptr;       /* the next pass records its Q8_0 activations here */
};

static int bfail(lg_bert* b, int rc)
{
    if (b && rc != LG_OK) snprintf(b->err, sizeof(b->err), "%s", lg_get_thread_error());
    return rc;
}

static int balloc(lg_bert* b, void** p, size_t bytes)
{
    const hipError_t e = hipMalloc(p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        lg_set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        return LG_ERR_NOMEM;
    }
    b->allocs.push_back(*p);
    return LG_OK;
}

static void bert_free_model(lg_bert* b)
{
    for (void* p : b->allocs) (void)hipFree(p);
    b->allocs.clear();
    b->layers.clear();
    if (b->meta_host) (void)hipHostFree(b->meta_host);
    if (b->emb_host) (void)hipHostFree(b->emb_host);
    b->meta_host = nullptr;
    b->emb_host = nullptr;
    b->loaded = false;
    b->vdb = nullptr;
    b->vdb_n = b->vdb_cap = 0;
}

extern "C" int lg_bert_create(int device, lg_bert** out)
{
    if (!out) { lg_set_error("lg_bert_create: null output"); return LG_ERR_ARG; }
    lg_rand_guard keep_rand;
    *out = nullptr;
    int n = 0;
    LG_HIP_CHECK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) { lg_set_error("lg_bert_create: device %d of %d", device, n); return LG_ERR_ARG; }
    LG_HIP_CHECK(hipSetDevice(device));
    lg_bert* b = new lg_bert();
    b->device = device;
    const hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        lg_set_error("hipStreamCreate failed: %s", hipGetErrorString(e));
        delete b;
        return LG_ERR_HIP;
    }
    *out = b;
    return LG_OK;
}

extern "C" int lg_bert_destroy(lg_bert* b)
{
    if (!b) return LG_OK;
    (void)hipSetDevice(b->device);
    (void)hipStreamSynchronize(b->stream);
    bert_free_model(b);
    if (b->vdb_out_host) (void)hipHostFree(b->vdb_out_host);
    (void)hipStreamDestroy(b->stream);
    delete b;
    return LG_OK;
}

extern "C" const char* lg_bert_last_error(const lg_bert* b) { return b ? b->err : lg_get_thread_error(); }

static bool q8_class(int t) { return t == LG_Q8_0 || t == LG_Q1_0 || t == LG_Q1_G; }
static int form_of(int t) { return q8_class(t) ? BF_I8 : t; }

static int bcheck_w(const lg_weight& w, int rows, int cols, const char* name)
{
    if (!w.data) { lg_set_error("bert load: %s missing", name); return LG_ERR_ARG; }
    if (w.rows != rows || w.cols != cols) {
        lg_set_error("bert load: %s is %dx%d, expected %dx%d", name, w.rows, w.cols, rows, cols);
        return LG_ERR_ARG;
    }
    if (w.type != LG_F32 && w.type != LG_F16 && !q8_class(w.type)) {
        lg_set_error("bert load: %s has type %d (F32, F16, Q8_0, Q1_0 or Q1_G)", name, w.type);
        return LG_ERR_TYPE;
    }
    if (w.type == LG_Q1_G && cols % 128) { lg_set_error("bert load: %s: Q1_G needs a multiple of 128 columns", name); return LG_ERR_ARG; }
    const int64_t need = lg_row_size(w.type, cols);
    if (need < 0 || (int64_t)w.rsz != need) {
        lg_set_error("bert load: %s row size %u (type %d rows of %d need %lld)", name, w.rsz, w.type, cols, (long long)need);
        return LG_ERR_ARG;
    }
    return LG_OK;
}

static int bput(lg_bert* b, void** dst, const void* src, size_t bytes)
{
    int rc = balloc(b, dst, bytes);
    if (rc) return rc;
    LG_HIP_CHECK(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
    return LG_OK;
}

static int bput_floats(lg_bert* b, float** dst, const float* src, size_t n, const char* name)
{
    if (!src) { lg_set_error("bert load: %s missing", name); return LG_ERR_ARG; }
    return bput(b, (void**)dst, src, n * sizeof(float));
}

/* upload matrices ws[0..n) (same form, same cols) stacked by rows into one */
static int bput_mat(lg_bert* b, const lg_weight* const* ws, int n, BMat& out)
{
    const int form = form_of(ws[0]->type), cols = ws[0]->cols;
    int rows = 0;
    for (int i = 0; i < n; i++) rows += ws[i]->rows;
    out.type = form;
    out.rows = rows;
    out.cols = cols;
    int rc;
    if (form != BF_I8) {
        const size_t esz = form == LG_F32 ? 4 : 2;
        if ((rc = balloc(b, (void**)&out.w, (size_t)rows * cols * esz))) return rc;
        size_t off = 0;
        for (int i = 0; i < n; i++) {
            const size_t bytes = (size_t)ws[i]->rows * ws[i]->rsz;
            LG_HIP_CHECK(hipMemcpy(out.w + off, ws[i]->data, bytes, hipMemcpyHostToDevice));
            off += bytes;
        }
        return LG_OK;
    }
    if ((rc = balloc(b, (void**)&out.w, (size_t)rows * cols))) return rc;
    if ((rc = balloc(b, (void**)&out.d, (size_t)rows * (cols / 32) * sizeof(float)))) return rc;
    int row_off = 0;
    for (int i = 0; i < n; i++) {
        const size_t bytes = (size_t)ws[i]->rows * ws[i]->rsz;
        uint8_t* tmp = nullptr;
        LG_HIP_CHECK(hipMalloc((void**)&tmp, bytes));
        hipError_t e = hipMemcpy(tmp, ws[i]->data, bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            const long work = (long)ws[i]->rows * (cols / 32);
            hipLaunchKernelGGL(k_bert_repack, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, b->stream,
                               ws[i]->type, (const uint8_t*)tmp, ws[i]->rsz, ws[i]->rows, cols, (int8_t*)out.w, out.d,
                               rows, row_off);
            e = hipGetLastError();
            if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
        }
        (void)hipFree(tmp);
        if (e != hipSuccess) { lg_set_error("bert load: repack: %s", hipGetErrorString(e)); return LG_ERR_HIP; }
        row_off += ws[i]->rows;
    }
    return LG_OK;
}

static int bert_load_impl(lg_bert* b, const lg_bert_desc* m, int max_tokens)
{
    const int ne = m->n_embed, nff = m->n_ff;
    if (m->n_layers < 0 || ne <= 0 || m->n_heads <= 0 || nff <= 0 || m->n_context < 2 || m->vocab_size <= 0 ||
        (m->n_layers > 0 && !m->layers)) {
        lg_set_error("bert load: bad model description");
        return LG_ERR_ARG;
    }
    if (ne % m->n_heads || ne % 32 || nff % 32 || ne > BERT_NE_MAX || nff > 4 * BERT_NE_MAX) {
        lg_set_error("bert load: n_embed %d / n_ff %d / heads %d unsupported (multiples of 32, n_embed <= %d)", ne, nff,
                     m->n_heads, BERT_NE_MAX);
        return LG_ERR_ARG;
    }
    const int hd = ne / m->n_heads;
    if (hd % 16 || hd > BERT_HD_MAX) { lg_set_error("bert load: head_dim %d (multiple of 16, <= %d)", hd, BERT_HD_MAX); return LG_ERR_ARG; }
    if (m->n_context > BERT_NCTX_MAX) { lg_set_error("bert load: n_context %d above %d", m->n_context, BERT_NCTX_MAX); return LG_ERR_ARG; }
    if (m->tok_cls < 0 || m->tok_cls >= m->vocab_size || m->tok_sep < 0 || m->tok_sep >= m->vocab_size) {
        lg_set_error("bert load: cls/sep ids %d/%d outside the vocabulary", m->tok_cls, m->tok_sep);
        return LG_ERR_ARG;
    }
    int rc;
    /* embedding tables: any row type lg_dq_value reads */
    const lg_weight* et[3] = {&m->tok_embd, &m->pos_embd, &m->tok_types};
    const int erows[3] = {m->vocab_size, m->n_context, 1};
    const char* en[3] = {"token_embd", "position_embd", "token_types"};
    for (int i = 0; i < 3; i++) {
        const lg_weight& w = *et[i];
        const int64_t need = lg_row_size(w.type, ne);
        if (!w.data || w.cols != ne || w.rows < erows[i] || need < 0 || (int64_t)w.rsz < need || w.type == LG_Q8_K) {
            lg_set_error("bert load: %s is %dx%d of type %d (needs >= %d rows of %d)", en[i], w.rows, w.cols, w.type,
                         erows[i], ne);
            return LG_ERR_ARG;
        }
    }
    b->n_layers = m->n_layers; b->ne = ne; b->nh = m->n_heads; b->hd = hd; b->nff = nff;
    b->nctx = m->n_context; b->vocab = m->vocab_size; b->tok_cls = m->tok_cls; b->tok_sep = m->tok_sep; b->eps = m->eps;
    b->tok_t = m->tok_embd.type; b->pos_t = m->pos_embd.type; b->typ_t = m->tok_types.type;
    b->tok_rsz = m->tok_embd.rsz; b->pos_rsz = m->pos_embd.rsz;
    if ((rc = bput(b, (void**)&b->tok, m->tok_embd.data, (size_t)m->vocab_size * m->tok_embd.rsz))) return rc;
    if ((rc = bput(b, (void**)&b->pos, m->pos_embd.data, (size_t)m->n_context * m->pos_embd.rsz))) return rc;
    if ((rc = bput(b, (void**)&b->typ, m->tok_types.data, m->tok_types.rsz))) return rc;
    if ((rc = bput_floats(b, &b->emb_w, m->emb_norm_w, ne, "token_embd_norm.weight"))) return rc;
    if ((rc = bput_floats(b, &b->emb_b, m->emb_norm_b, ne, "token_embd_norm.bias"))) return rc;

    b->layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        const lg_bert_layer_desc& L = m->layers[l];
        BLayer& D = b->layers[l];
        if ((rc = bcheck_w(L.attn_q, ne, ne, "attn_q")) || (rc = bcheck_w(L.attn_k, ne, ne, "attn_k")) ||
            (rc = bcheck_w(L.attn_v, ne, ne, "attn_v")) || (rc = bcheck_w(L.attn_out, ne, ne, "attn_output")) ||
            (rc = bcheck_w(L.ffn_up, nff, ne, "ffn_up")) || (rc = bcheck_w(L.ffn_down, ne, nff, "ffn_down")))
            return rc;
        const lg_weight* qkv[3] = {&L.attn_q, &L.attn_k, &L.attn_v};
        if (form_of(L.attn_q.type) == form_of(L.attn_k.type) && form_of(L.attn_q.type) == form_of(L.attn_v.type)) {
            D.nqkv = 1;
            if ((rc = bput_mat(b, qkv, 3, D.qkv[0]))) return rc;
        } else {
            D.nqkv = 3;
            for (int i = 0; i < 3; i++)
                if ((rc = bput_mat(b, qkv + i, 1, D.qkv[i]))) return rc;
        }
        const lg_weight* ao = &L.attn_out;
        const lg_weight* up = &L.ffn_up;
        const lg_weight* dn = &L.ffn_down;
        if ((rc = bput_mat(b, &ao, 1, D.ao)) || (rc = bput_mat(b, &up, 1, D.up)) || (rc = bput_mat(b, &dn, 1, D.down)))
            return rc;
        if (!L.attn_q_bias || !L.attn_k_bias || !L.attn_v_bias) { lg_set_error("bert load: layer %d: q/k/v bias missing", l); return LG_ERR_ARG; }
        std::vector<float> bq(3 * (size_t)ne);
        memcpy(bq.data(), L.attn_q_bias, ne * sizeof(float));
        memcpy(bq.data() + ne, L.attn_k_bias, ne * sizeof(float));
        memcpy(bq.data() + 2 * ne, L.attn_v_bias, ne * sizeof(float));
        if ((rc = bput_floats(b, &D.qkv_bias, bq.data(), 3 * (size_t)ne, "attn_qkv.bias")) ||
            (rc = bput_floats(b, &D.ao_bias, L.attn_out_bias, ne, "attn_output.bias")) ||
            (rc = bput_floats(b, &D.ln1_w, L.attn_norm_w, ne, "attn_output_norm.weight")) ||
            (rc = bput_floats(b, &D.ln1_b, L.attn_norm_b, ne, "attn_output_norm.bias")) ||
            (rc = bput_floats(b, &D.up_bias, L.ffn_up_bias, nff, "ffn_up.bias")) ||
            (rc = bput_floats(b, &D.down_bias, L.ffn_down_bias, ne, "ffn_down.bias")) ||
            (rc = bput_floats(b, &D.ln2_w, L.ffn_norm_w, ne, "layer_output_norm.weight")) ||
            (rc = bput_floats(b, &D.ln2_b, L.ffn_norm_b, ne, "layer_output_norm.bias")))
            return rc;
    }

    /* activations for tmax tokens */
    int tmax = max_tokens > 0 ? max_tokens : std::max(m->n_context, 4096);
    if (tmax < m->n_context) { lg_set_error("bert load: max_tokens %d below n_context %d", tmax, m->n_context); return LG_ERR_ARG; }
    tmax = (tmax + 63) & ~63;
    b->tmax = tmax;
    b->ldd = tmax;
    const size_t T = tmax, wmax = std::max(ne, nff);
    if ((rc = balloc(b, (void**)&b->x, T * ne * 4)) || (rc = balloc(b, (void**)&b->x1, T * ne * 4)) ||
        (rc = balloc(b, (void**)&b->y, T * ne * 4)) || (rc = balloc(b, (void**)&b->qkv, T * 3 * ne * 4)) ||
        (rc = balloc(b, (void**)&b->ctx, T * ne * 4)) || (rc = balloc(b, (void**)&b->h, T * nff * 4)) ||
        (rc = balloc(b, (void**)&b->aq, T * wmax)) || (rc = balloc(b, (void**)&b->ad, T * (wmax / 32) * 4)) ||
        (rc = balloc(b, (void**)&b->emb_dev, (T / 2) * ne * 4)) || (rc = balloc(b, (void**)&b->q_emb_dev, (size_t)ne * 4)))
        return rc;
    /* tables: tokpos T int2, attention blocks (<= T/4 + T/2) x 4 ints, sequences T/2 int2 */
    b->meta_bytes = T * 8 + (T / 4 + T / 2 + 1) * sizeof(BAttnBlk) + (T / 2) * 8;
    if ((rc = balloc(b, &b->meta_dev, b->meta_bytes))) return rc;
    LG_HIP_CHECK(hipHostMalloc((void**)&b->meta_host, b->meta_bytes, 0));
    LG_HIP_CHECK(hipHostMalloc((void**)&b->emb_host, (T / 2) * ne * 4, 0));
    if ((rc = balloc(b, (void**)&b->vdb_cand, (size_t)VDB_BLOCKS_MAX * LG_VDB_KMAX * 8)) ||
        (rc = balloc(b, (void**)&b->vdb_out, (1 + 2 * LG_VDB_KMAX) * 4)))
        return rc;
    if (!b->vdb_out_host) LG_HIP_CHECK(hipHostMalloc((void**)&b->vdb_out_host, (1 + 2 * LG_VDB_KMAX) * 4, 0));
    b->loaded = true;
    return LG_OK;
}

extern "C" int lg_bert_load(lg_bert* b, const lg_bert_desc* desc, int max_tokens)
{
    if (!b || !desc) { lg_set_error("lg_bert_load: null argument"); return bfail(b, LG_ERR_ARG); }
    (void)hipSetDevice(b->device);
    (void)hipStreamSynchronize(b->stream);
    bert_free_model(b);
    const int rc = bert_load_impl(b, desc, max_tokens);
    if (rc) bert_free_model(b);
    return bfail(b, rc);
}

/* ---- one pass ---- */
template <int WT, int EP, int TM, int TN>
static void gemm_launch(const BGemm& a, hipStream_t s)
{
    const dim3 grid((unsigned)(((a.T + 16 * TM - 1) / (16 * TM)) * ((a.R + 16 * TN - 1) / (16 * TN))));
    hipLaunchKernelGGL((k_bert_gemm<WT, EP, TM, TN>), grid, dim3(64), 0, s, a);
}

template <int WT, int EP>
static void gemm_tiles(const BGemm& a, hipStream_t s)
{
    /* the largest wave tile whose grid still has ~3 waves per SIMD */
    auto waves = [&](int tm, int tn) { return (long)((a.T + 16 * tm - 1) / (16 * tm)) * ((a.R + 16 * tn - 1) / (16 * tn)); };
    if (waves(2, 2) >= 3072) gemm_launch<WT, EP, 2, 2>(a, s);
    else if (waves(1, 2) >= 3072) gemm_launch<WT, EP, 1, 2>(a, s);
    else gemm_launch<WT, EP, 1, 1>(a, s);
}

template <int EP>
static int gemm_ep(const BMat& W, const float* x, int ldx, const lg_bert* b, int T, const float* bias, const float* res,
                   int ldr, float* out, int ldo)
{
    BGemm a;
    a.w = W.w; a.wd = W.d; a.R = W.rows; a.K = W.cols;
    a.x = x; a.ldx = ldx; a.q = b->aq; a.qd = b->ad; a.ldd = b->ldd;
    a.T = T; a.bias = bias; a.res = res; a.ldr = ldr; a.out = out; a.ldo = ldo;
    switch (W.type) {
    case LG_F32: gemm_tiles<LG_F32, EP>(a, b->stream); break;
    case LG_F16: gemm_tiles<LG_F16, EP>(a, b->stream); break;
    default: gemm_tiles<BF_I8, EP>(a, b->stream); break;
    }
    return lg_check_launch("bert gemm");
}

/* The same GEMM for the batched prefill's F32/F16 layer matrices
 * (lg_prefill.h): out[t][r] (+)= W[r] . x[t], fp32 activations. */
int lg_fgemm_tokens(int wtype, const uint8_t* W, int rows, int cols, const float* x, int ldx, int T, float* out, int ldo,
                    int accumulate, hipStream_t s)
{
    if ((wtype != LG_F32 && wtype != LG_F16) || !W || !x || !out || rows <= 0 || cols <= 0 || cols % 32 || T <= 0 ||
        ldx < cols || ldx % 4 || ldo < rows) {
        lg_set_error("fp gemm: bad arguments (type %d, rows %d, cols %d, T %d)", wtype, rows, cols, T);
        return LG_ERR_ARG;
    }
    BGemm a = {};
    a.w = W; a.R = rows; a.K = cols; a.x = x; a.ldx = ldx; a.T = T; a.out = out; a.ldo = ldo;
    if (wtype == LG_F32) {
        if (accumulate) gemm_tiles<LG_F32, EP_ADD>(a, s);
        else gemm_tiles<LG_F32, EP_STORE>(a, s);
    } else {
        if (accumulate) gemm_tiles<LG_F16, EP_ADD>(a, s);
        else gemm_tiles<LG_F16, EP_STORE>(a, s);
    }
    return lg_check_launch("fp gemm");
}

static int launch_quant(const lg_bert* b, const float* x, int n, int T)
{
    hipLaunchKernelGGL(k_bert_quant, dim3(T), dim3(256), 0, b->stream, x, n, b->aq, b->ad, b->ldd);
    return lg_check_launch("bert quant");
}

static int launch_ln(const lg_bert* b, const float* y, const float* w, const float* bias, float* out, bool quant, int T)
{
    const int np = (b->ne + 1023) / 1024;
    int8_t* q = quant ? b->aq : nullptr;
#define LN_CASE(NP) \
    case NP: hipLaunchKernelGGL(k_bert_ln<NP>, dim3(T), dim3(256), 0, b->stream, y, b->ne, w, bias, b->eps, out, q, b->ad, b->ldd); break
    switch (np) {
        LN_CASE(1); LN_CASE(2); LN_CASE(3); LN_CASE(4);
    default: lg_set_error("bert: n_embed %d", b->ne); return LG_ERR_ARG;
    }
#undef LN_CASE
    return lg_check_launch("bert layernorm");
}

/* activation trace: slot (layer, point) holds int8 [T][K] then, at
 * tmax * wmax, the scales [K/32][T] */
static size_t trace_slot_bytes(const lg_bert* b)
{
    const size_t w = (size_t)std::max(b->ne, b->nff);
    return (size_t)b->tmax * w + (w / 32) * b->tmax * 4;
}

static int trace_copy(const lg_bert* b, int l, int s, int K, int T)
{
    if (!b->trace) return LG_OK;
    uint8_t* dst = b->trace + ((size_t)l * 4 + s) * trace_slot_bytes(b);
    LG_HIP_CHECK(hipMemcpyAsync(dst, b->aq, (size_t)T * K, hipMemcpyDeviceToDevice, b->stream));
    LG_HIP_CHECK(hipMemcpy2DAsync(dst + (size_t)b->tmax * std::max(b->ne, b->nff), (size_t)T * 4, b->ad,
                                  (size_t)b->ldd * 4, (size_t)T * 4, (size_t)K / 32, hipMemcpyDeviceToDevice, b->stream));
    return LG_OK;
}

static bool any_i8(const BLayer& L)
{
    for (int i = 0; i < L.nqkv; i++)
        if (L.qkv[i].type == BF_I8) return true;
    return false;
}

/* the encoder over the T tokens whose tables are in meta_dev */
static int bert_layers(lg_bert* b, int T, int nblk, int qb, int pst, int nseq)
{
    const int ne = b->ne;
    const int2* tokpos = (const int2*)b->meta_dev;
    const BAttnBlk* blks = (const BAttnBlk*)((uint8_t*)b->meta_dev + (size_t)b->tmax * 8);
    const int2* seqs = (const int2*)((uint8_t*)blks + ((size_t)b->tmax / 4 + b->tmax / 2 + 1) * sizeof(BAttnBlk));
    int rc;
    {
        BEmbArgs a;
        a.tok = b->tok; a.pos = b->pos; a.typ = b->typ;
        a.tok_t = b->tok_t; a.pos_t = b->pos_t; a.typ_t = b->typ_t;
        a.tok_rsz = b->tok_rsz; a.pos_rsz = b->pos_rsz;
        a.tokpos = tokpos; a.w = b->emb_w; a.b = b->emb_b; a.eps = b->eps; a.n = ne; a.out = b->x;
        a.q = (b->n_layers > 0 && any_i8(b->layers[0])) ? b->aq : nullptr;
        a.qd = b->ad; a.ldd = b->ldd;
        switch ((ne + 1023) / 1024) {
        case 1: hipLaunchKernelGGL(k_bert_embed<1>, dim3(T), dim3(256), 0, b->stream, a); break;
        case 2: hipLaunchKernelGGL(k_bert_embed<2>, dim3(T), dim3(256), 0, b->stream, a); break;
        case 3: hipLaunchKernelGGL(k_bert_embed<3>, dim3(T), dim3(256), 0, b->stream, a); break;
        default: hipLaunchKernelGGL(k_bert_embed<4>, dim3(T), dim3(256), 0, b->stream, a); break;
        }
        if ((rc = lg_check_launch("bert embed"))) return rc;
        if (a.q && (rc = trace_copy(b, 0, 0, ne, T))) return rc;
    }
    const float scale = 1.0f / sqrtf((float)b->hd);
    for (int l = 0; l < b->n_layers; l++) {
        const BLayer& L = b->layers[l];
        /* q|k|v = W x + bias (fast/vdb.cpp:180-186) */
        if (L.nqkv == 1) {
            if ((rc = gemm_ep<EP_BIAS>(L.qkv[0], b->x, ne, b, T, L.qkv_bias, nullptr, 0, b->qkv, 3 * ne))) return rc;
        } else {
            /* mixed forms: x's Q8_0 (if any of them needs it) came with x */
            for (int i = 0; i < 3; i++)
                if ((rc = gemm_ep<EP_BIAS>(L.qkv[i], b->x, ne, b, T, L.qkv_bias + i * ne, nullptr, 0, b->qkv + i * ne, 3 * ne)))
                    return rc;
        }
        /* attention (fast/vdb.cpp:189-212) */
        const dim3 ag((unsigned)nblk, (unsigned)b->nh);
#define ATT_CASE(HD)                                                                                                  \
    case HD:                                                                                                          \
        if (pst <= 128)                                                                                               \
            hipLaunchKernelGGL((k_bert_attn_mfma<HD, 128>), ag, dim3(256), 0, b->stream, b->qkv, ne, blks, scale, b->ctx); \
        else if (pst <= 256)                                                                                          \
            hipLaunchKernelGGL((k_bert_attn_mfma<HD, 256>), ag, dim3(256), 0, b->stream, b->qkv, ne, blks, scale, b->ctx); \
        else if (pst <= 512)                                                                                          \
            hipLaunchKernelGGL((k_bert_attn_mfma<HD, 512>), ag, dim3(256), 0, b->stream, b->qkv, ne, blks, scale, b->ctx); \
        else if (pst <= 1024)                                                                                         \
            hipLaunchKernelGGL((k_bert_attn_mfma<HD, 1024>), ag, dim3(256), 0, b->stream, b->qkv, ne, blks, scale, b->ctx); \
        else                                                                                                          \
            hipLaunchKernelGGL(k_bert_attn<HD>, ag, dim3(256), 0, b->stream, b->qkv, ne, blks, qb, pst, scale, b->ctx); \
        break
        switch (b->hd) {
            ATT_CASE(16); ATT_CASE(32); ATT_CASE(48); ATT_CASE(64); ATT_CASE(80); ATT_CASE(96); ATT_CASE(112); ATT_CASE(128);
        default: lg_set_error("bert: head_dim %d", b->hd); return LG_ERR_ARG;
        }
#undef ATT_CASE
        if ((rc = lg_check_launch("bert attention"))) return rc;
        /* x1 = layernorm(att_out ctx + bias + x) (fast/vdb.cpp:219-222) */
        if (L.ao.type == BF_I8 && ((rc = launch_quant(b, b->ctx, ne, T)) || (rc = trace_copy(b, l, 1, ne, T)))) return rc;
        if ((rc = gemm_ep<EP_BIAS_RES>(L.ao, b->ctx, ne, b, T, L.ao_bias, b->x, ne, b->y, ne))) return rc;
        if ((rc = launch_ln(b, b->y, L.ln1_w, L.ln1_b, b->x1, L.up.type == BF_I8, T))) return rc;
        if (L.up.type == BF_I8 && (rc = trace_copy(b, l, 2, ne, T))) return rc;
        /* h = gelu(up x1 + bias); x = layernorm(down h + bias + x1) (:224-231) */
        if ((rc = gemm_ep<EP_BIAS_GELU>(L.up, b->x1, ne, b, T, L.up_bias, nullptr, 0, b->h, b->nff))) return rc;
        if (L.down.type == BF_I8 && ((rc = launch_quant(b, b->h, b->nff, T)) || (rc = trace_copy(b, l, 3, b->nff, T))))
            return rc;
        if ((rc = gemm_ep<EP_BIAS_RES>(L.down, b->h, b->nff, b, T, L.down_bias, b->x1, ne, b->y, ne))) return rc;
        const bool qn = l + 1 < b->n_layers && any_i8(b->layers[l + 1]);
        if ((rc = launch_ln(b, b->y, L.ln2_w, L.ln2_b, b->x, qn, T))) return rc;
        if (qn && (rc = trace_copy(b, l + 1, 0, ne, T))) return rc;
    }
    hipLaunchKernelGGL(k_bert_pool_mean, dim3(nseq, (ne + 63) / 64), dim3(1024), 0, b->stream, b->x, ne, seqs,
                       b->emb_dev);
    if ((rc = lg_check_launch("bert pool"))) return rc;
    hipLaunchKernelGGL(k_bert_l2norm, dim3(nseq), dim3(256), 0, b->stream, b->emb_dev, ne);
    return lg_check_launch("bert l2norm");
}

/* the attention query block for the longest sequence of a pass */
static int attn_qb(int nmax) { return nmax <= 1024 ? 16 : nmax <= 2048 ? 8 : 4; }

/* Embed sequences [s_begin, s_end) of (toks, offsets) in one pass; the
 * caller has checked that their wrapped lengths fit tmax. */
static int bert_pass(lg_bert* b, const int* toks, const int* offsets, int s_begin, int s_end, float* out_host)
{
    const int nseq = s_end - s_begin;
    int2* tokpos = (int2*)b->meta_host;
    BAttnBlk* blks = (BAttnBlk*)(b->meta_host + (size_t)b->tmax * 8);
    int2* seqs = (int2*)((uint8_t*)blks + ((size_t)b->tmax / 4 + b->tmax / 2 + 1) * sizeof(BAttnBlk));
    int nmax = 0;
    for (int s = s_begin; s < s_end; s++) nmax = std::max(nmax, std::min(offsets[s + 1] - offsets[s], b->nctx - 2) + 2);
    const int qb = attn_qb(nmax);
    const int pst = (nmax + 63) & ~63;
    int T = 0, nblk = 0;
    for (int s = s_begin; s < s_end; s++) {
        const int raw = std::min(offsets[s + 1] - offsets[s], b->nctx - 2);   /* toks.resize(n_context - 2) */
        const int n = raw + 2;
        tokpos[T] = make_int2(b->tok_cls, 0);
        for (int i = 0; i < raw; i++) tokpos[T + 1 + i] = make_int2(toks[offsets[s] + i], 1 + i);
        tokpos[T + n - 1] = make_int2(b->tok_sep, n - 1);
        for (int q = 0; q < n; q += qb) blks[nblk++] = BAttnBlk{T + q, std::min(qb, n - q), T, n};
        seqs[s - s_begin] = make_int2(T, n);
        T += n;
    }
    for (int i = 0; i < T; i++)
        if (tokpos[i].x < 0 || tokpos[i].x >= b->vocab) {
            lg_set_error("bert embed: token %d outside the vocabulary of %d", tokpos[i].x, b->vocab);
            return LG_ERR_ARG;
        }
    LG_HIP_CHECK(hipMemcpyAsync(b->meta_dev, b->meta_host, b->meta_bytes, hipMemcpyHostToDevice, b->stream));
    int rc = bert_layers(b, T, nblk, qb, pst, nseq);
    b->trace = nullptr;                                  /* one pass only */
    if (rc) return rc;
    if (out_host) {
        LG_HIP_CHECK(hipMemcpyAsync(b->emb_host, b->emb_dev, (size_t)nseq * b->ne * 4, hipMemcpyDeviceToHost, b->stream));
        LG_HIP_CHECK(hipStreamSynchronize(b->stream));
        memcpy(out_host, b->emb_host, (size_t)nseq * b->ne * 4);
    } else {
        LG_HIP_CHECK(hipStreamSynchronize(b->stream));   /* the host tables are rewritten by the next pass */
    }
    return LG_OK;
}

static int embed_batch(lg_bert* b, const int* toks, const int* offsets, int nseq, float* out_host)
{
    if (!b->loaded) { lg_set_error("bert: no model loaded"); return LG_ERR_STATE; }
    if (!toks && offsets && nseq > 0 && offsets[nseq] > offsets[0]) { lg_set_error("bert embed: null tokens"); return LG_ERR_ARG; }
    for (int s = 0; s < nseq; s++)
        if (offsets[s + 1] < offsets[s]) { lg_set_error("bert embed: offsets decrease at %d", s); return LG_ERR_ARG; }
    LG_HIP_CHECK(hipSetDevice(b->device));
    int s0 = 0;
    while (s0 < nseq) {
        int T = 0, s1 = s0;
        while (s1 < nseq) {
            const int n = std::min(offsets[s1 + 1] - offsets[s1], b->nctx - 2) + 2;
            if (T + n > b->tmax || s1 - s0 >= b->tmax / 2) break;
            T += n;
            s1++;
        }
        const int rc = bert_pass(b, toks, offsets, s0, s1, out_host ? out_host + (size_t)s0 * b->ne : nullptr);
        if (rc) return rc;
        s0 = s1;
    }
    return LG_OK;
}

extern "C" int lg_bert_embed(lg_bert* b, const int* toks, int ntok, float* out_host)
{
    if (!b || ntok < 0 || (ntok > 0 && !toks) || !out_host) { lg_set_error("lg_bert_embed: bad arguments"); return bfail(b, LG_ERR_ARG); }
    const int off[2] = {0, ntok};
    return bfail(b, embed_batch(b, toks, off, 1, out_host));
}

extern "C" int lg_bert_embed_batch(lg_bert* b, const int* toks, const int* offsets, int nseq, float* out_host)
{
    if (!b || nseq < 0 || (nseq > 0 && (!offsets || !out_host))) {
        lg_set_error("lg_bert_embed_batch: bad arguments");
        return bfail(b, LG_ERR_ARG);
    }
    return bfail(b, embed_batch(b, toks, offsets, nseq, out_host));
}

extern "C" size_t lg_bert_trace_size(const lg_bert* b)
{
    return b && b->loaded ? (size_t)b->n_layers * 4 * trace_slot_bytes(b) : 0;
}

extern "C" int lg_bert_trace_next(lg_bert* b, void* trace_dev)
{
    if (!b) { lg_set_error("lg_bert_trace_next: null handle"); return LG_ERR_ARG; }
    if (!b->loaded) { lg_set_error("bert: no model loaded"); return bfail(b, LG_ERR_STATE); }
    b->trace = (uint8_t*)trace_dev;
    return LG_OK;
}

/* ---- vector memory ---- */
static int vdb_reserve(lg_bert* b, int n)
{
    if (n <= b->vdb_cap) return LG_OK;
    int cap = std::max(n, std::max(1024, 2 * b->vdb_cap));
    uint16_t* nv = nullptr;
    const hipError_t e = hipMalloc((void**)&nv, (size_t)cap * b->ne * 2);
    if (e != hipSuccess) { lg_set_error("vdb: hipMalloc(%zu): %s", (size_t)cap * b->ne * 2, hipGetErrorString(e)); return LG_ERR_NOMEM; }
    if (b->vdb_n) LG_HIP_CHECK(hipMemcpyAsync(nv, b->vdb, (size_t)b->vdb_n * b->ne * 2, hipMemcpyDeviceToDevice, b->stream));
    LG_HIP_CHECK(hipStreamSynchronize(b->stream));
    if (b->vdb) {
        (void)hipFree(b->vdb);
        b->allocs.erase(std::find(b->allocs.begin(), b->allocs.end(), (void*)b->vdb));
    }
    b->vdb = nv;
    b->allocs.push_back(nv);
    b->vdb_cap = cap;
    return LG_OK;
}

static int vdb_put(lg_bert* b, const uint16_t* vecs, int n, int dim, bool replace)
{
    if (!b->loaded) { lg_set_error("vdb: no encoder loaded"); return LG_ERR_STATE; }
    if (n < 0 || (n > 0 && !vecs) || dim != b->ne) { lg_set_error("vdb: %d rows of %d (the encoder's width is %d)", n, dim, b->ne); return LG_ERR_ARG; }
    LG_HIP_CHECK(hipSetDevice(b->device));
    const int base = replace ? 0 : b->vdb_n;
    int rc = vdb_reserve(b, base + n);
    if (rc) return rc;
    if (n) LG_HIP_CHECK(hipMemcpy(b->vdb + (size_t)base * dim, vecs, (size_t)n * dim * 2, hipMemcpyHostToDevice));
    b->vdb_n = base + n;
    return LG_OK;
}

extern "C" int lg_bert_vdb_set(lg_bert* b, const uint16_t* vecs_host, int n, int dim)
{
    if (!b) { lg_set_error("lg_bert_vdb_set: null handle"); return LG_ERR_ARG; }
    return bfail(b, vdb_put(b, vecs_host, n, dim, true));
}

extern "C" int lg_bert_vdb_append(lg_bert* b, const uint16_t* vecs_host, int n, int dim)
{
    if (!b) { lg_set_error("lg_bert_vdb_append: null handle"); return LG_ERR_ARG; }
    return bfail(b, vdb_put(b, vecs_host, n, dim, false));
}

extern "C" int lg_bert_vdb_size(const lg_bert* b) { return b ? b->vdb_n : -1; }

/* search with the embedding at emb_dev (device); results to the host */
static int vdb_search(lg_bert* b, const float* emb_dev, float threshold, int k, int* idx_out, float* sim_out)
{
    if (k <= 0 || k > LG_VDB_KMAX) { lg_set_error("vdb query: k %d (1..%d)", k, LG_VDB_KMAX); return LG_ERR_ARG; }
    if (b->vdb_n == 0) return 0;
    const int per_block = 4 * 8;
    const int nb = std::min(VDB_BLOCKS_MAX, (b->vdb_n + per_block - 1) / per_block);
    hipLaunchKernelGGL(k_vdb_search, dim3(nb), dim3(256), 0, b->stream, b->vdb, b->vdb_n, b->ne, emb_dev, threshold, k,
                       b->vdb_cand);
    int rc = lg_check_launch("vdb search");
    if (rc) return rc;
    hipLaunchKernelGGL(k_vdb_merge, dim3(1), dim3(256), 0, b->stream, (const uint64_t*)b->vdb_cand, nb * k, k, b->vdb_out);
    if ((rc = lg_check_launch("vdb merge"))) return rc;
    LG_HIP_CHECK(hipMemcpyAsync(b->vdb_out_host, b->vdb_out, (1 + 2 * LG_VDB_KMAX) * 4, hipMemcpyDeviceToHost, b->stream));
    LG_HIP_CHECK(hipStreamSynchronize(b->stream));
    const int cnt = b->vdb_out_host[0];
    for (int r = 0; r < cnt; r++) {
        if (idx_out) idx_out[r] = b->vdb_out_host[1 + r];
        if (sim_out) memcpy(&sim_out[r], &b->vdb_out_host[1 + LG_VDB_KMAX + r], 4);
    }
    return cnt;
}

extern "C" int lg_bert_vdb_query(lg_bert* b, const float* emb_host, int dim, float threshold, int k, int* idx_out,
                                 float* sim_out)
{
    if (!b || !emb_host) { lg_set_error("lg_bert_vdb_query: bad arguments"); return bfail(b, LG_ERR_ARG); }
    if (!b->loaded) { lg_set_error("vdb: no encoder loaded"); return bfail(b, LG_ERR_STATE); }
    if (dim != b->ne) { lg_set_error("vdb query: dim %d, the encoder's width is %d", dim, b->ne); return bfail(b, LG_ERR_ARG); }
    (void)hipSetDevice(b->device);
    const hipError_t e = hipMemcpy(b->q_emb_dev, emb_host, (size_t)dim * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) { lg_set_error("vdb query: %s", hipGetErrorString(e)); return bfail(b, LG_ERR_HIP); }
    return bfail(b, vdb_search(b, b->q_emb_dev, threshold, k, idx_out, sim_out));
}

extern "C" int lg_bert_query(lg_bert* b, const int* toks, int ntok, float threshold, int k, int* idx_out,
                             float* sim_out, float* emb_out_host)
{
    if (!b || ntok < 0 || (ntok > 0 && !toks)) { lg_set_error("lg_bert_query: bad arguments"); return bfail(b, LG_ERR_ARG); }
    if (k <= 0 || k > LG_VDB_KMAX) { lg_set_error("lg_bert_query: k %d (1..%d)", k, LG_VDB_KMAX); return bfail(b, LG_ERR_ARG); }
    const int off[2] = {0, ntok};
    int rc = embed_batch(b, toks, off, 1, emb_out_host);
    if (rc) return bfail(b, rc);
    return bfail(b, vdb_search(b, b->emb_dev, threshold, k, idx_out, sim_out));
}
