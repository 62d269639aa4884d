/* lg_prefill.hip -- feed_text's prompt loop (fast/ligguf_fast_qk.cpp:340-356)
 * as layer passes over T tokens at once.  Each token's arithmetic is that of
 * inference() (:24-144); what changes is that every weight matrix is read
 * once per pass and multiplied by the T quantized activations with int8
 * MFMA:
 *   - activations are quantized per token as the decode step does (same
 *     rmsnorm lane order, same Q8_K quantizer, lg_q8k_lane);
 *   - Q4_K x Q8_K (fast/lil_math.cpp:582-616): the integer sum of q*a of
 *     each 32-value sub-block is one v_mfma_i32_16x16x32_i8 (K = 32), exact;
 *     S = sum_j sc_j * isum_j in int32, exact; the mins term
 *     M = sum_j m_j * (bsums[2j] + bsums[2j+1]) is a K = 8 product on
 *     v_mfma_f32_16x16x4f32, exact (every partial sum is an integer below
 *     2^24); then out += d_a * (d_w * S - dmin_w * M) per 256-value block;
 *   - attention per query token over the fp16 cache rows before it and its
 *     own fp32 k/v (:64-105), after the pass has written the KV rows of all
 *     its tokens;
 * so every integer of the reference's decomposition is reproduced and only
 * the fp32 accumulation order differs from T sequential steps. */
#include <math.h>
#include <type_traits>

#include "lg_common.h"
#include "lg_fmt.h"
#include "lg_prefill.h"
#include "lg_quant.h"
#include "lg_rope.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef short v2i16 __attribute__((ext_vector_type(2)));

template <typename To, typename From>
__device__ __forceinline__ To lg_bits(From v)
{
    static_assert(sizeof(To) == sizeof(From), "same size");
    To t;
    __builtin_memcpy(&t, &v, sizeof(To));
    return t;
}

/* ------------------------------------------------------------------ */
/* embedding rows, quantizers                                           */
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(256) void k_pf_embed(int type, const uint8_t* __restrict__ table, uint32_t rsz,
                                                  const int* __restrict__ toks, int n, float* __restrict__ x)
{
    const int t = blockIdx.x;
    const uint8_t* row = table + (size_t)toks[t] * rsz;
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[(size_t)t * n + i] = lg_dq_value(type, row, i);
}

/* one 256-value block of one token into the SoA Q8_K form */
__device__ __forceinline__ void pf_store_q8k(const float v[4], const PfQ8K& q, int n, int t, int b)
{
    const int lane = threadIdx.x & 63;
    const Q8KLane r = lg_q8k_lane(v);
    *(uint32_t*)(q.qs + (size_t)t * n + b * 256 + 4 * lane) = r.packed;
    if ((lane & 3) == 0) q.bs[((size_t)t * (n >> 8) + b) * 16 + (lane >> 2)] = (int16_t)r.bsum;
    if (lane == 0) q.d[(size_t)b * q.tld + t] = r.d;
}

/* one 256-value chunk of one token as eight Q8_0 blocks in the SoA form:
 * qs as the Q8_K form, d [K/32][tld] the fp16 scale as the reference
 * stores it (read back as float), asum [K/32][tld] the blocks' sums of q */
__device__ __forceinline__ void pf_store_q8_0(const float v[4], const PfQ8K& q, int n, int t, int b)
{
    const int lane = threadIdx.x & 63;
    const Q80Lane r = lg_q8_0_lane(v);
    /* the block's sum of q over its 8 lanes: integers below 2^24, exact in fp32 */
    const int bs = (int)lg_group_sum<8>((float)lg_dot4((int)r.packed, 0x01010101, 0));
    if (b * 256 + 4 * lane >= n) return;   /* blocks past a width that is no multiple of 256 (8 lanes each) */
    *(uint32_t*)(q.qs + (size_t)t * n + b * 256 + 4 * lane) = r.packed;
    if ((lane & 7) == 0) {
        const size_t i = (size_t)(8 * b + (lane >> 3)) * q.tld + t;
        q.d[i] = lg_h2f(lg_f2h(r.d));
        q.as[i] = bs;
    }
}

template <int QT>
__device__ __forceinline__ void pf_store(const float v[4], const PfQ8K& q, int n, int t, int b)
{
    if constexpr (QT == LG_Q8_K) pf_store_q8k(v, q, n, t, b);
    else if constexpr (QT == LG_Q8_0) pf_store_q8_0(v, q, n, t, b);
    else {
        /* the fp32 values (F32/F16 weights take them unquantized) */
        const int i = b * 256 + 4 * (threadIdx.x & 63);
        if (i < n) *(float4*)(q.f + (size_t)t * n + i) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

/* token t (one workgroup of 4 waves): rmsnorm(x_t) * w (w != NULL) or
 * x_t, quantized (Q8_K or Q8_0) block by block, wave w taking blocks w,
 * w + 4, ...  The sum of squares in the decode kernels' order
 * (lg_sumsq_chunked, fast/lil_math.cpp:922-929): eight 2048-strided chunk
 * sets, each one wave sum, added in set order -- here sets v and v + 4 by
 * wave v, the eight sums through LDS -- computed once per token. */
template <int QT>
__global__ __launch_bounds__(256) void k_pf_quant(const float* __restrict__ x, int ldx, const float* __restrict__ w,
                                                  float eps, int n, PfQ8K q)
{
    __shared__ float s_ss[8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = blockIdx.x;
    const float* xr = x + (size_t)t * ldx;
    float scale = 1.0f;
    if (w) {
        for (int v = wave; v < 8; v += 4) {
            float p = 0.0f;
            for (int i = 256 * v + 4 * lane; i < n; i += 2048) p += lg_sq4(*(const float4*)(xr + i));
            const float sv = lg_wave_sum(p);
            if (lane == 0) s_ss[v] = sv;
        }
        __syncthreads();
        float ss = 0.0f;
        for (int v = 0; v < 8; v++) ss += s_ss[v];
        scale = 1.0f / sqrtf(ss / (float)n + eps);
    }
    const int nb = (n + 255) / 256;
    for (int b = wave; b < nb; b += 4) {
        const int base = b * 256 + 4 * lane;
        const bool in = base < n;   /* Q8_0 widths that are no multiple of 256: zeros past the end, not stored */
        const float4 tv = in ? *(const float4*)(xr + base) : make_float4(0.f, 0.f, 0.f, 0.f);
        float v[4] = {tv.x, tv.y, tv.z, tv.w};
        if (w && in) {
            const float4 g = *(const float4*)(w + base);
            v[0] = tv.x * scale * g.x; v[1] = tv.y * scale * g.y; v[2] = tv.z * scale * g.z; v[3] = tv.w * scale * g.w;
        }
        pf_store<QT>(v, q, n, t, b);
    }
}

/* hb = silu(gate) * up of token t (fast/ligguf_fast_qk.cpp:119-123), block b,
 * quantized; ug row = [up | gate] */
template <int QT>
__global__ __launch_bounds__(64) void k_pf_swiglu_quant(const float* __restrict__ ug, int nff, PfQ8K q)
{
    const int lane = threadIdx.x, b = blockIdx.x, t = blockIdx.y;
    const float* ur = ug + (size_t)t * 2 * nff;
    const int base = b * 256 + 4 * lane;
    const bool in = base < nff;
    const float4 u = in ? *(const float4*)(ur + base) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 g = in ? *(const float4*)(ur + nff + base) : make_float4(0.f, 0.f, 0.f, 0.f);
    float v[4];
    v[0] = (g.x / (1.0f + expf(-g.x))) * u.x;
    v[1] = (g.y / (1.0f + expf(-g.y))) * u.y;
    v[2] = (g.z / (1.0f + expf(-g.z))) * u.z;
    v[3] = (g.w / (1.0f + expf(-g.w))) * u.w;
    pf_store<QT>(v, q, nff, t, b);
}

/* QK-norm + RoPE + KV rows of token t at position pos0 + t */
__global__ __launch_bounds__(256) void k_pf_qk_rope_kv(float* __restrict__ qkv, int qstride, int n_embed, int kv_dim,
                                                       const float* __restrict__ qw, const float* __restrict__ kw,
                                                       int n_heads, int n_kv, int hd, int rope_dim, int pos0,
                                                       const float* __restrict__ freq, float eps,
                                                       uint16_t* __restrict__ kc, uint16_t* __restrict__ vc)
{
    const int t = blockIdx.y;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int pos = pos0 + t;
    float* q = qkv + (size_t)t * qstride;
    lg_qk_norm_rope_kv_wave(wave, q, q + n_embed, q + n_embed + kv_dim, qw, kw, n_heads, n_kv, hd, rope_dim, pos,
                            freq, eps, kc + (size_t)pos * kv_dim, vc + (size_t)pos * kv_dim);
}

/* ------------------------------------------------------------------ */
/* Q4_K x Q8_K GEMM on int8 MFMA                                        */
/* ------------------------------------------------------------------ */
/* Workgroup tile: 16 MI tokens x 128 rows, 8 waves of 16 MI tokens x 16
 * rows (MI MFMA tiles of 16 x 16 per wave: a wave's weight operands,
 * unpacked once per sub-block pair, feed 2 MI MFMAs).  v_mfma_i32_16x16x64_i8
 * (checked on the part; twice the rate of the K = 32 form, 4.5 against 2.3
 * int8 POP/s): lane l holds 16 bytes of A[token l%16] and of B[.][row l%16]
 * for lane group l/16, and D[token 4(l/16)+i][row l%16] in register i.
 * In a Q4_K block, byte 32c+i of qs holds value 64c+i (low nibble) and
 * 64c+32+i (high nibble), so lane group g takes bytes 32c+8g..+7 of its
 * row: the low nibbles are its 8 values of sub-block 2c, the high ones of
 * sub-block 2c+1; the activation bytes 64c+8g and 64c+32+8g match them.
 *
 * S = sum_j sc_j isum_j over the 8 sub-blocks with sc_j = 8 h_j + l_j
 * (h, l < 8): the weights scaled by h_j and by l_j still fit int8
 * (q h <= 105), so both sums accumulate inside the MFMA over the whole
 * block and S = 8 S_h + S_l exactly, with no per-sub-block readback.  A
 * packed 16-bit multiply scales four q bytes at once (every product is
 * below 256, so no carry crosses a byte).
 *
 * Per 256-value block the token tile's quants, bsums and block scales are
 * staged in LDS (double-buffered, rows padded to 272 B against bank
 * conflicts, quants reordered per lane group) and shared by the 8 waves; each wave reads its rows' bytes
 * straight from the GGUF rows, one block ahead.  Rows and tokens past the
 * ends are clamped for the loads and not stored.  The grid is one
 * dimension: (row block, token tile) from the index, XCD-aware. */
#ifndef LG_PF_NT
#define LG_PF_NT 512
#endif
#define PF_NT LG_PF_NT         /* threads per workgroup */
#define PF_RB (PF_NT / 4)      /* rows per workgroup: waves of 16 */
#define PF_AST 272             /* LDS row stride of the staged quants */
/* MI token tiles of 16 per workgroup */
template <int ACC, int MI>
__global__ __launch_bounds__(PF_NT) __attribute__((amdgpu_waves_per_eu(4))) void k_pf_gemm_q4k(const uint8_t* __restrict__ W, uint32_t rsz, int R, int K,
                                                     PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    __shared__ __attribute__((aligned(16))) int8_t s_a[2][(16 * MI) * PF_AST];
    __shared__ __attribute__((aligned(16))) int16_t s_bs[2][(16 * MI) * 16];
    __shared__ __attribute__((aligned(16))) float s_d[2][(16 * MI)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int nb = K >> 8;
    /* tile of this workgroup: workgroups go to the 8 XCDs round-robin by
     * index, so the token tiles of one row block get indices 8 apart -- one
     * XCD, dispatched together -- and its weight bytes come from HBM once
     * and from that XCD's L2 for the other token tiles */
    const int nt = (T + (16 * MI) - 1) / (16 * MI);
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * PF_RB >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * (16 * MI);
    const int r0 = rb * PF_RB + wave * 16;
    const uint8_t* wr = W + (size_t)min(r0 + l16, R - 1) * rsz;

    /* staging, per block: thread tid takes quant chunks tid + 512 i (token
     * chunk/16, 16-byte piece chunk%16), one 8-byte quarter of a token's
     * bsums (token tid/4, threads < 64 MI) and, threads < 4 MI, four block
     * scales */
    constexpr int NA = MI * 256 / PF_NT;   /* quant chunks per thread: 16 MI tokens x 16 / threads */
    struct Stg {
        uint4 a[NA];
        uint2 bs;
        uint4 d;
    };
    auto stage_load = [&](Stg& st, int b) {
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int q = tid + PF_NT * i, tok = min(t0 + (q >> 4), T - 1);
            st.a[i] = *(const uint4*)(x.qs + (size_t)tok * K + (size_t)b * 256 + (q & 15) * 16);
        }
        const int tb = min(t0 + ((tid >> 2) & (16 * MI - 1)), T - 1);
        st.bs = *(const uint2*)(x.bs + ((size_t)tb * nb + b) * 16 + (tid & 3) * 4);
        st.d = *(const uint4*)(x.d + (size_t)b * x.tld + min(t0 + 4 * (tid & (4 * MI - 1)), x.tld - 4));
    };
    /* LDS order of a token's 256 quants: for each 64-value chunk c and lane
     * group g, the 8 values 64c + 8g.. then the 8 values 64c + 32 + 8g.. --
     * the 16 bytes one lane feeds to a K = 64 product, read with one
     * conflict-free ds_read_b128.  Piece p = 4c + k of the row (bytes
     * 64c + 16k..+15) holds the first halves of groups 2(k&1), 2(k&1)+1 (k
     * < 2) or their second halves (k >= 2). */
    auto stage_store = [&](const Stg& st, int buf) {
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int q = tid + PF_NT * i, p = q & 15, k = p & 3;
            int8_t* d = s_a[buf] + (q >> 4) * PF_AST + 64 * (p >> 2) + 32 * (k & 1) + 8 * (k >> 1);
            *(uint2*)d = make_uint2(st.a[i].x, st.a[i].y);
            *(uint2*)(d + 16) = make_uint2(st.a[i].z, st.a[i].w);
        }
        if (tid < 64 * MI) *(uint2*)(s_bs[buf] + (tid >> 2) * 16 + (tid & 3) * 4) = st.bs;
        if (tid < 4 * MI) *(uint4*)(s_d[buf] + 4 * tid) = st.d;
    };
    /* the wave's weight operands of one block */
    struct Blk {
        uint4 hdr;
        uint2 wq[4];
    };
    auto blk_load = [&](Blk& B, int b) {
        const uint8_t* p = wr + (size_t)b * LG_BS_Q4_K;
        B.hdr = *(const uint4*)p;
#pragma unroll
        for (int c = 0; c < 4; c++) B.wq[c] = *(const uint2*)(p + 16 + 32 * c + 8 * g);
    };

    v4f acc[MI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++) acc[mi] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int b, const Blk& cur) {
        const int buf = b & 1;
        /* scales of the lane's row (get_scale_min_k4, fast/lil_math.cpp:129-138) */
        const uint4 h4 = cur.hdr;
        const uint32_t scq[2] = {h4.y & 0x3F3F3F3Fu, (h4.w & 0x0F0F0F0Fu) | ((h4.y >> 2) & 0x30303030u)};
        const uint32_t mlo = h4.z & 0x3F3F3F3Fu;
        const uint32_t mhi = ((h4.w >> 4) & 0x0F0F0F0Fu) | ((h4.z >> 2) & 0x30303030u);
        const float mb0 = (float)((mlo >> (8 * g)) & 0xFFu);   /* m_j, j = g */
        const float mb1 = (float)((mhi >> (8 * g)) & 0xFFu);   /* m_j, j = g + 4 */
        const float dw = lg_h2f((uint16_t)(h4.x & 0xffffu));
        const float dmw = lg_h2f((uint16_t)(h4.x >> 16));
        v4i Sh[MI], Sl[MI];
#pragma unroll
        for (int mi = 0; mi < MI; mi++) Sh[mi] = Sl[mi] = (v4i){0, 0, 0, 0};
        const int8_t* sa = s_a[buf] + l16 * PF_AST + 16 * g;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            /* one K = 64 product per chunk c: bytes 0-7 of a lane are its 8
             * values of sub-block 2c (low nibbles), bytes 8-15 those of
             * sub-block 2c+1 (high nibbles), against the matching activation
             * bytes 64c + 8g and 64c + 32 + 8g (the MFMA pairs byte i of A's
             * lane group with byte i of B's, whatever k it stands for) */
            v4i bh, bl;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int j = 2 * c + h;
                const uint2 q = cur.wq[c];
                const uint32_t lo = h ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
                const uint32_t hi = h ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
                const uint32_t sc = (scq[j >> 2] >> (8 * (j & 3))) & 0x3Fu;
                const v2u16 sh = (v2u16)(uint16_t)(sc >> 3), sl = (v2u16)(uint16_t)(sc & 7u);
                bh[2 * h] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(lo) * sh);
                bh[2 * h + 1] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(hi) * sh);
                bl[2 * h] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(lo) * sl);
                bl[2 * h + 1] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(hi) * sl);
            }
#pragma unroll
            for (int mi = 0; mi < MI; mi++) {
                const uint4 a = *(const uint4*)(sa + 16 * mi * PF_AST + 64 * c);
                const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                Sh[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bh, Sh[mi], 0, 0, 0);
                Sl[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bl, Sl[mi], 0, 0, 0);
            }
        }
        /* mins term M[token][row] = sum_j m_j (bsums_2j + bsums_2j+1) on the
         * fp32 MFMA (k = g: sub-blocks g and g + 4), and the block's fp32
         * contribution acc += d_a (d_w S - dmin_w M) */
#pragma unroll
        for (int mi = 0; mi < MI; mi++) {
            const int16_t* bsr = s_bs[buf] + (16 * mi + l16) * 16;
            const int v0 = *(const int*)(bsr + 2 * g), v1 = *(const int*)(bsr + 2 * (g + 4));
            const float bpa0 = (float)((int)(int16_t)(v0 & 0xffff) + (int)(int16_t)(v0 >> 16));
            const float bpa1 = (float)((int)(int16_t)(v1 & 0xffff) + (int)(int16_t)(v1 >> 16));
            v4f M = __builtin_amdgcn_mfma_f32_16x16x4f32(bpa0, mb0, (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            M = __builtin_amdgcn_mfma_f32_16x16x4f32(bpa1, mb1, M, 0, 0, 0);
            const float4 dx = *(const float4*)(s_d[buf] + 16 * mi + 4 * g);
            const v4i S = Sh[mi] * 8 + Sl[mi];
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
                acc[mi][i] = __builtin_fmaf(dxs[i], lg_fma2(dw, (float)S[i], -dmw, M[i]), acc[mi][i]);
        }
    };

    /* one block ahead: block b+1's operands load while block b computes */
    Blk cur, nxt;
    Stg st;
    stage_load(st, 0);
    blk_load(cur, 0);
    stage_store(st, 0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int bn = min(b + 1, nb - 1);
        stage_load(st, bn);
        blk_load(nxt, bn);
        compute(b, cur);
        stage_store(st, (b + 1) & 1);
        cur = nxt;
        __syncthreads();
    }
    const int r = r0 + l16;
#pragma unroll
    for (int mi = 0; mi < MI; mi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * mi + 4 * g + i;
            if (t < T && r < R) {
                float* o = out + (size_t)t * ldo + r;
                *o = ACC ? *o + acc[mi][i] : acc[mi][i];
            }
        }
    }
}

/* The same products on the 32 x 32 forms: v_mfma_i32_32x32x32_i8 takes 16
 * bytes of a 32-row A and of a 32-column B per lane, twice the multiplies
 * of a 16x16x64 product per operand byte, so each token fragment read from
 * LDS feeds twice the work.  A workgroup of 4 waves computes 128 rows x 64
 * tokens, a wave 32 rows x 64 tokens (two 32 x 32 tiles, token rows i,
 * weight columns j): lane l holds row j = l % 32 of its wave's rows and the
 * K bytes 16 (l / 32) .. +15 of a 32-value sub-block -- sub-block 2c is the
 * low nibbles and 2c+1 the high nibbles of the same 16 bytes of qs --
 * against the token's quants 32s + 16 (l / 32) .. +15, read from its LDS
 * row as stored; C register r of lane l is token 8 (r / 4) + 4 (l / 32) +
 * r % 4 of the tile, row l % 32.  Scales split sc = 8h + l as in
 * k_pf_gemm_q4k (two products per sub-block, S = 8 S_h + S_l exactly).
 * The mins term M = sum_s m_s (bsums_2s + bsums_2s+1) is one
 * v_mfma_f32_32x32x16_f16 per tile: each pair sum p = 64 p_hi + p_lo is
 * staged as two fp16 integers (p_hi in [-64, 63], p_lo in [0, 63]) against
 * 64 m_s and m_s, so every product and partial sum is an integer below
 * 2^24 and M is exact.  Then out += d_a (d_w S - dmin_w M) per block in the
 * same fp32 operations as k_pf_gemm_q4k, so both give the same bits.
 *
 * Q5_K rows (WT = LG_Q5_K): the Q4_K layout of scales and mins with a
 * fifth bit per value from qh; w = sc q < 2^11 is formed in 16-bit halves
 * and split w = 64 w_h + w_l (w_h <= 30, w_l <= 63), S = 64 S_h + S_l, and
 * the mins term and the fp32 operations are Q4_K's (k_pf_gemm_kq's Q5_K
 * dot gives the same bits).
 *
 * Q6_K rows (WT = LG_Q6_K) on the same tile: lane l's 16 bytes of chunk s
 * (values 32s + 16 (l / 32) ..) are the whole of 16-value sub-block
 * 2s + l / 32, so the lane folds its scale into them: w = sc (q - 32) (sc
 * the int8 scale, |w| <= 4096, one packed 16-bit multiply-add per two
 * values) is split w = 64 w_h + w_l (w_h in [-64, 64], w_l in [0, 63]) and
 * the two byte forms go through two products: S = 64 S_h + S_l =
 * sum_i sc_i sum (q - 32) a, the integer of k_pf_gemm_kq's Q6_K dot,
 * exactly; out += (d_w d_a) S as there, so the two kernels give the same
 * bits. */
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
#define PF2_NT 256
#define PF2_RB 128    /* rows per workgroup */
#define PF2_AST 272   /* LDS row stride of a token's 256 quants */
/* KS = 2 (the 4096-row att_out and down products, whose 128 x 64 tiles
 * alone would leave one wave per SIMD): 8 waves, waves 4..7 take the second
 * half of K with LDS stages of their own, and their sums are added to the
 * first half's through LDS at the end (acc0 + acc1, one fixed order) */
template <int WT, int ACC, int KS>
__global__ __launch_bounds__(PF2_NT * KS) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gemm_k32(
    const uint8_t* __restrict__ W, uint32_t rsz, int R, int K, PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    static_assert(WT == LG_Q2_K || WT == LG_Q3_K || WT == LG_Q4_K || WT == LG_Q5_K || WT == LG_Q6_K || WT == LG_Q6_K_R,
                  "K-quant rows");
    /* LG_Q6_K_R: the fused decode step's regrouped Q6_K rows (per run of 8
     * blocks: their ql, qh, scales, d), the same values at aligned offsets */
    /* the mins term: Q4_K and Q5_K (32-value sub-blocks: pair sums of the
     * bsums, split 64 p_hi + p_lo) or Q2_K (16-value sub-blocks: the bsums) */
    constexpr int MK = (WT == LG_Q4_K || WT == LG_Q5_K) ? 1 : WT == LG_Q2_K ? 2 : 0;
    constexpr bool MINS = MK != 0;
    constexpr int BSZ = WT == LG_Q2_K ? LG_BS_Q2_K : WT == LG_Q3_K ? LG_BS_Q3_K : WT == LG_Q4_K ? LG_BS_Q4_K
                      : WT == LG_Q5_K ? LG_BS_Q5_K : LG_BS_Q6_K;
    constexpr int TT = 64;   /* tokens per workgroup: two 32-token tiles per wave */
    __shared__ __attribute__((aligned(16))) int8_t s_a[KS][2][TT * PF2_AST];
    /* per token: p_hi[8], p_lo[8] or the 16 bsums (the mins term) */
    constexpr int MST = MINS ? TT * 16 : 8;
    __shared__ __attribute__((aligned(16))) _Float16 s_m[KS][2][MST];
    __shared__ __attribute__((aligned(16))) float s_d[KS][2][TT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kh = wave >> 2, tid = threadIdx.x & (PF2_NT - 1);   /* K half; thread within it */
    const int h = lane >> 5, j = lane & 31;
    const int nb = K >> 8;
    /* this half's blocks b0 .. b0 + nbh - 1; every wave runs L steps */
    const int nb0 = KS == 2 ? (nb + 1) / 2 : nb;
    const int b0 = kh * nb0, nbh = kh ? nb - nb0 : nb0, L = nb0;
    const int nt = (T + TT - 1) / TT;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * PF2_RB >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * TT;
    const int row = rb * PF2_RB + (wave & 3) * 32 + j;
    const uint8_t* wr = W + (size_t)min(row, R - 1) * rsz;
    int8_t(*sa_)[TT * PF2_AST] = s_a[kh];
    _Float16(*sm_)[MST] = s_m[kh];
    float(*sd_)[TT] = s_d[kh];

    /* staging, per block: quant chunk q = tid + 256 u (token q / 16, piece
     * q % 16); thread tid also takes bsums 4 (tid % 4) .. +3 of token tid / 4
     * (pair sums 2 (tid % 4), +1) and, tid < 64, the d of token tid */
    struct Stg {   /* clang vectors, not HIP's uint4 structs: their copies stay in registers */
        v4i a[4];
        uint2 bs;
        float d;
    };
    auto stage_load = [&](Stg& st, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = tid + PF2_NT * u, tok = min(t0 + (q >> 4), T - 1);
            st.a[u] = *(const v4i*)(x.qs + (size_t)tok * K + (size_t)b * 256 + (q & 15) * 16);
        }
        if constexpr (MINS) {   /* the bsums feed the mins term */
            const int tb = min(t0 + (tid >> 2), T - 1);
            st.bs = *(const uint2*)(x.bs + ((size_t)tb * nb + b) * 16 + (tid & 3) * 4);
        }
        st.d = x.d[(size_t)b * x.tld + min(t0 + (tid & 63), x.tld - 1)];
    };
    auto stage_store = [&](const Stg& st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = tid + PF2_NT * u;
            *(v4i*)(sa_[buf] + (q >> 4) * PF2_AST + (q & 15) * 16) = st.a[u];
        }
        const int tok = tid >> 2;   /* bsums / mins of token tid / 4 */
        if constexpr (MK == 2) {
            const v4h m = {(_Float16)(float)(int16_t)(st.bs.x & 0xffff), (_Float16)(float)(int16_t)(st.bs.x >> 16),
                           (_Float16)(float)(int16_t)(st.bs.y & 0xffff), (_Float16)(float)(int16_t)(st.bs.y >> 16)};
            *(v4h*)(sm_[buf] + tok * 16 + 4 * (tid & 3)) = m;
        } else if constexpr (MINS) {
            const int s0 = 2 * (tid & 3);
            const int p0 = (int)(int16_t)(st.bs.x & 0xffff) + (int)(int16_t)(st.bs.x >> 16);
            const int p1 = (int)(int16_t)(st.bs.y & 0xffff) + (int)(int16_t)(st.bs.y >> 16);
            _Float16* m = sm_[buf] + tok * 16;
            m[s0] = (_Float16)(float)(p0 >> 6);
            m[s0 + 1] = (_Float16)(float)(p1 >> 6);
            m[8 + s0] = (_Float16)(float)(p0 & 63);
            m[8 + s0 + 1] = (_Float16)(float)(p1 & 63);
        }
        if (tid < 64) sd_[buf][tid] = st.d;
    };
    /* the lane's weight bytes of one block: Q4_K the header and 4 x 16 B of
     * qs; Q6_K 4 x 16 B of ql, 2 x 16 B of qh, the 16 scales and d */
    struct Blk4 {
        uint4 hdr;
        uint4 q[4];
    };
    struct Blk5 {
        uint4 hdr;
        uint4 q[4];
        v4i qh;
    };
    struct Blk6 {
        v4i ql[4], qh[2], sc;
        uint32_t d;
    };
    struct Blk2 {
        v4i qs[2], sc;
        uint32_t dd;
    };
    struct Blk3 {
        v4i hm, qs[2];
        uint32_t s0, s1, s2, d;
    };
    using Blk = typename std::conditional<
        WT == LG_Q4_K, Blk4,
        typename std::conditional<
            WT == LG_Q5_K, Blk5,
            typename std::conditional<WT == LG_Q6_K || WT == LG_Q6_K_R, Blk6,
                                      typename std::conditional<WT == LG_Q2_K, Blk2, Blk3>::type>::type>::type>::type;
    auto blk_load = [&](Blk& B, int b) __attribute__((always_inline)) {
        const uint8_t* p = wr + (size_t)b * BSZ;
        if constexpr (WT == LG_Q4_K) {
            B.hdr = *(const uint4*)p;
#pragma unroll
            for (int c = 0; c < 4; c++) B.q[c] = *(const uint4*)(p + 16 + 32 * c + 16 * h);
        } else if constexpr (WT == LG_Q2_K) {
            /* 84-byte blocks: scales[16], qs[64], d, dmin */
            B.sc = lg_ld<v4i>(p);
            B.qs[0] = lg_ld<v4i>(p + 16 + 16 * h);
            B.qs[1] = lg_ld<v4i>(p + 48 + 16 * h);
            B.dd = lg_ld<uint32_t>(p + 80);
        } else if constexpr (WT == LG_Q3_K) {
            /* 110-byte blocks: hmask[32], qs[64], scales[12], d */
            B.hm = lg_ld<v4i>(p + 16 * h);
            B.qs[0] = lg_ld<v4i>(p + 32 + 16 * h);
            B.qs[1] = lg_ld<v4i>(p + 64 + 16 * h);
            B.s0 = lg_ld<uint32_t>(p + 96);
            B.s1 = lg_ld<uint32_t>(p + 100);
            B.s2 = lg_ld<uint32_t>(p + 104);
            B.d = lg_ld16(p + 108);
        } else if constexpr (WT == LG_Q5_K) {
            /* 176-byte blocks: 16-byte aligned */
            B.hdr = *(const uint4*)p;
            B.qh = *(const v4i*)(p + 16 + 16 * h);
#pragma unroll
            for (int c = 0; c < 4; c++) B.q[c] = *(const uint4*)(p + 48 + 32 * c + 16 * h);
        } else if constexpr (WT == LG_Q6_K_R) {
            const uint8_t* g = wr + (size_t)(b >> 3) * 8 * LG_BS_Q6_K;
            const int e = b & 7;
#pragma unroll
            for (int n = 0; n < 2; n++) {
                B.ql[2 * n] = *(const v4i*)(g + 128 * e + 64 * n + 16 * h);
                B.ql[2 * n + 1] = *(const v4i*)(g + 128 * e + 64 * n + 32 + 16 * h);
                B.qh[n] = *(const v4i*)(g + 1024 + 64 * e + 32 * n + 16 * h);
            }
            B.sc = *(const v4i*)(g + 1536 + 16 * e);
            B.d = lg_ld16(g + 1664 + 2 * e);
        } else {
            /* 210-byte blocks: 2-byte aligned (unaligned dword loads) */
#pragma unroll
            for (int n = 0; n < 2; n++) {
                B.ql[2 * n] = lg_ld<v4i>(p + 64 * n + 16 * h);
                B.ql[2 * n + 1] = lg_ld<v4i>(p + 64 * n + 32 + 16 * h);
                B.qh[n] = lg_ld<v4i>(p + 128 + 32 * n + 16 * h);
            }
            B.sc = lg_ld<v4i>(p + 192);
            B.d = lg_ld16(p + 208);
        }
    };

    v16f acc[2];
    acc[0] = (v16f){};
    acc[1] = (v16f){};

    auto compute6 = [&](int buf, const Blk6& cur) __attribute__((always_inline)) {
        const float dw = lg_h2f((uint16_t)cur.d);
        v16i Sh[2], Sl[2];
#pragma unroll
        for (int t = 0; t < 2; t++) Sh[t] = Sl[t] = (v16i){};
        const int8_t* sa = sa_[buf] + j * PF2_AST + 16 * h;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            /* chunk s = values 128 n + 64 c + 32 e + (0..31): nibble c of
             * ql[64 n + 32 e + ..], bits 2 (2c + e) of qh[32 n + ..] */
            const int n = s >> 2, c = (s >> 1) & 1, e = s & 1, sb = 2 * s + h;
            const v4i ql = cur.ql[2 * n + e], qh = cur.qh[n];
            const int sc = (int)(int8_t)(cur.sc[sb >> 2] >> (8 * (sb & 3)));
            const v2i16 sc2 = (v2i16)(short)sc, off2 = (v2i16)(short)(-32 * sc);
            v4i bh, bl;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t q = (((uint32_t)ql[k] >> (4 * c)) & 0x0F0F0F0Fu) |
                                   ((((uint32_t)qh[k] >> (2 * (2 * c + e))) & 0x03030303u) << 4);
                /* values 0, 2 and 1, 3 in 16-bit halves: w = sc q - 32 sc,
                 * then w_h = w >> 6 and w_l = w & 63 back to bytes */
                const v2i16 we = lg_bits<v2i16>(q & 0x00FF00FFu) * sc2 + off2;
                const v2i16 wo = lg_bits<v2i16>(__builtin_amdgcn_perm(0u, q, 0x0C030C01u)) * sc2 + off2;   /* bytes 1, 3 */
                const uint32_t he = lg_bits<uint32_t>((v2i16)(we >> (short)6)),
                               ho = lg_bits<uint32_t>((v2i16)(wo >> (short)6));
                /* v_perm_b32 selector 0x06020400: bytes 0, 2 of the second
                 * operand interleaved with bytes 0, 2 of the first */
                bh[k] = (int)__builtin_amdgcn_perm(ho, he, 0x06020400u);
                bl[k] = (int)(__builtin_amdgcn_perm(lg_bits<uint32_t>(wo), lg_bits<uint32_t>(we), 0x06020400u) & 0x3F3F3F3Fu);
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * s);
                const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                Sh[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bh, Sh[t], 0, 0, 0);
                Sl[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bl, Sl[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v16i S = Sh[t] * 64 + Sl[t];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dx = *(const float4*)(sd_[buf] + 32 * t + 8 * g + 4 * h);
                const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g + i;
                    acc[t][r] = __builtin_fmaf(dw * dxs[i], (float)S[r], acc[t][r]);
                }
            }
        }
    };
    /* Q2_K: w = sc q <= 45 (bytes, two to a 16-bit multiply), one product
     * per chunk; the mins term sum_i m_i bsums_i is one
     * v_mfma_f32_32x32x16_f16 per tile (|bsum| <= 2048, m <= 15: exact) */
    auto compute2 = [&](int buf, const Blk2& cur) __attribute__((always_inline)) {
        const float dw = lg_h2f((uint16_t)(cur.dd & 0xffffu)), dmw = lg_h2f((uint16_t)(cur.dd >> 16));
        v8h bm;   /* mins of sub-blocks 8h .. 8h + 7 */
#pragma unroll
        for (int k = 0; k < 8; k++) bm[k] = (_Float16)(float)(((uint32_t)cur.sc[2 * h + (k >> 2)] >> (8 * (k & 3) + 4)) & 15u);
        v16i S[2];
#pragma unroll
        for (int t = 0; t < 2; t++) S[t] = (v16i){};
        const int8_t* sa = sa_[buf] + j * PF2_AST + 16 * h;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            /* chunk s = values 128 n + 32 jj + (0..31): bits 2 jj of qs[32 n + ..] */
            const int n = s >> 2, jj = s & 3, sb = 2 * s + h;
            const v2u16 sc2 = (v2u16)(uint16_t)(((uint32_t)cur.sc[sb >> 2] >> (8 * (sb & 3))) & 15u);
            v4i bw;
#pragma unroll
            for (int k = 0; k < 4; k++)
                bw[k] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(((uint32_t)cur.qs[n][k] >> (2 * jj)) & 0x03030303u) * sc2);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * s);
                const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                S[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bw, S[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v8h am = *(const v8h*)(sm_[buf] + (32 * t + j) * 16 + 8 * h);
            const v16f M = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, (v16f){}, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dx = *(const float4*)(sd_[buf] + 32 * t + 8 * g + 4 * h);
                const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g + i;
                    acc[t][r] = __builtin_fmaf(dxs[i], lg_fma2(dw, (float)S[t][r], -dmw, M[r]), acc[t][r]);
                }
            }
        }
    };
    /* Q3_K: u = 2 bits of qs | the hmask bit << 2, value u - 4, scale sc =
     * 6 bits - 32; w = -sc (u - 4) in [-128, 124] fits a byte (sc (u - 4)
     * reaches 128), one product per chunk and S = -S' */
    auto compute3 = [&](int buf, const Blk3& cur) __attribute__((always_inline)) {
        const float dw = lg_h2f((uint16_t)cur.d);
        v16i S[2];
#pragma unroll
        for (int t = 0; t < 2; t++) S[t] = (v16i){};
        const int8_t* sa = sa_[buf] + j * PF2_AST + 16 * h;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int n = s >> 2, jj = s & 3, sb = 2 * s + h;
            /* scale sb: low nibble of byte sb (sb < 8) or high nibble of
             * byte sb - 8 of the first 8, two high bits from byte 8 + sb % 4
             * at 2 (sb / 4) */
            const uint32_t lw = (sb & 7) < 4 ? cur.s0 : cur.s1;
            const int lo = (int)((lw >> (8 * (sb & 3) + (sb < 8 ? 0 : 4))) & 15u);
            const int hi = (int)((cur.s2 >> (8 * (sb & 3) + 2 * (sb >> 2))) & 3u);
            const int sc = (lo | (hi << 4)) - 32;
            const v2i16 ws2 = (v2i16)(short)(-sc), off2 = (v2i16)(short)(4 * sc);
            v4i bw;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t u = (((uint32_t)cur.qs[n][k] >> (2 * jj)) & 0x03030303u) |
                                   ((((uint32_t)cur.hm[k] >> (4 * n + jj)) & 0x01010101u) << 2);
                const v2i16 we = lg_bits<v2i16>(u & 0x00FF00FFu) * ws2 + off2;
                const v2i16 wo = lg_bits<v2i16>(__builtin_amdgcn_perm(0u, u, 0x0C030C01u)) * ws2 + off2;
                bw[k] = (int)__builtin_amdgcn_perm(lg_bits<uint32_t>(wo), lg_bits<uint32_t>(we), 0x06020400u);
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * s);
                const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                S[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bw, S[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dx = *(const float4*)(sd_[buf] + 32 * t + 8 * g + 4 * h);
                const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g + i;
                    acc[t][r] = __builtin_fmaf(dw * dxs[i], (float)(-S[t][r]), acc[t][r]);
                }
            }
        }
    };
    auto compute = [&](int buf, const Blk& cur) __attribute__((always_inline)) {
      if constexpr (WT == LG_Q6_K || WT == LG_Q6_K_R) {
        compute6(buf, cur);
      } else if constexpr (WT == LG_Q2_K) {
        compute2(buf, cur);
      } else if constexpr (WT == LG_Q3_K) {
        compute3(buf, cur);
      } else {
        const uint4 h4 = cur.hdr;
        const uint32_t scq[2] = {h4.y & 0x3F3F3F3Fu, (h4.w & 0x0F0F0F0Fu) | ((h4.y >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {h4.z & 0x3F3F3F3Fu, ((h4.w >> 4) & 0x0F0F0F0Fu) | ((h4.z >> 2) & 0x30303030u)};
        const float dw = lg_h2f((uint16_t)(h4.x & 0xffffu));
        const float dmw = lg_h2f((uint16_t)(h4.x >> 16));
        /* mins operand: 64 m_s (lanes 0..31) or m_s (32..63), s = 0..7 */
        v8h bm;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int m = (int)((mn[s >> 2] >> (8 * (s & 3))) & 0xFFu);
            bm[s] = (_Float16)(float)(h ? m : 64 * m);
        }
        v16i Sh[2], Sl[2];
#pragma unroll
        for (int t = 0; t < 2; t++) Sh[t] = Sl[t] = (v16i){};
        const int8_t* sa = sa_[buf] + j * PF2_AST + 16 * h;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t qw[4] = {cur.q[c].x, cur.q[c].y, cur.q[c].z, cur.q[c].w};
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int s = 2 * c + e;
                const uint32_t sc = (scq[s >> 2] >> (8 * (s & 3))) & 0x3Fu;
                v4i bh, bl;
                if constexpr (WT == LG_Q4_K) {
                    const v2u16 sh = (v2u16)(uint16_t)(sc >> 3), sl = (v2u16)(uint16_t)(sc & 7u);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t nib = e ? (qw[k] >> 4) & 0x0F0F0F0Fu : qw[k] & 0x0F0F0F0Fu;
                        bh[k] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(nib) * sh);
                        bl[k] = (int)lg_bits<uint32_t>(lg_bits<v2u16>(nib) * sl);
                    }
                } else {
                    /* Q5_K: q = nibble e of qs | bit s of qh << 4 (0..31);
                     * w = sc q < 2^11 in 16-bit halves, w = 64 w_h + w_l */
                    const v2u16 sc2 = (v2u16)(uint16_t)sc;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t q = ((e ? qw[k] >> 4 : qw[k]) & 0x0F0F0F0Fu) |
                                           ((((uint32_t)cur.qh[k] >> s) & 0x01010101u) << 4);
                        const v2u16 we = lg_bits<v2u16>(q & 0x00FF00FFu) * sc2;
                        const v2u16 wo = lg_bits<v2u16>(__builtin_amdgcn_perm(0u, q, 0x0C030C01u)) * sc2;
                        const uint32_t he = lg_bits<uint32_t>((v2u16)(we >> (unsigned short)6)),
                                       ho = lg_bits<uint32_t>((v2u16)(wo >> (unsigned short)6));
                        bh[k] = (int)__builtin_amdgcn_perm(ho, he, 0x06020400u);
                        bl[k] = (int)(__builtin_amdgcn_perm(lg_bits<uint32_t>(wo), lg_bits<uint32_t>(we), 0x06020400u) &
                                      0x3F3F3F3Fu);
                    }
                }
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * s);
                    const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                    Sh[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bh, Sh[t], 0, 0, 0);
                    Sl[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bl, Sl[t], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v8h am = *(const v8h*)(sm_[buf] + (32 * t + j) * 16 + 8 * h);
            const v16f M = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, (v16f){}, 0, 0, 0);
            const v16i S = Sh[t] * (WT == LG_Q4_K ? 8 : 64) + Sl[t];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dx = *(const float4*)(sd_[buf] + 32 * t + 8 * g + 4 * h);
                const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g + i;
                    acc[t][r] = __builtin_fmaf(dxs[i], lg_fma2(dw, (float)S[r], -dmw, M[r]), acc[t][r]);
                }
            }
        }
      }
    };

    /* step i of this half: the token tile of block b0 + i + 2 loads into
     * registers while block b0 + i computes, and goes to LDS after it (two
     * blocks' compute for each staging load; one for the weights) */
    auto blk = [&](int i) { return b0 + min(i, nbh - 1); };
    Blk cur, nxt;
    Stg st0, st1;
    stage_load(st0, blk(0));
    stage_load(st1, blk(1));
    blk_load(cur, blk(0));
    stage_store(st0, 0);
    __syncthreads();
#define PF2_STEP(ii, ST_LD, ST_ST)                \
    do {                                          \
        stage_load(ST_LD, blk((ii) + 2));         \
        blk_load(nxt, blk((ii) + 1));             \
        if ((ii) < nbh) compute((ii) & 1, cur);   \
        stage_store(ST_ST, ((ii) + 1) & 1);       \
        cur = nxt;                                \
        __syncthreads();                          \
    } while (0)
    /* pairs of steps (an odd count ends on one that computes nothing; the
     * second half may have one block fewer) */
    for (int i = 0; i < L; i += 2) {
        PF2_STEP(i, st0, st1);
        PF2_STEP(i + 1, st1, st0);
    }
#undef PF2_STEP
    if constexpr (KS == 2) {
        /* the second half's sums through LDS (its stage buffers are done) */
        float* red = (float*)s_a[1];
        if (kh == 1) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[(t * 16 + r) * (PF2_NT) + tid] = acc[t][r];
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][r] = acc[t][r] + red[(t * 16 + r) * (PF2_NT) + tid];
    }
    if (row < R) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int tok = t0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                if (tok < T) {
                    float* o = out + (size_t)tok * ldo + row;
                    *o = ACC ? *o + acc[t][r] : acc[t][r];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */
/* LG_PF_GEMM16=1: the 16 x 16 product kernels for the K-quant, Q8_0 and
 * Q1_0 rows */
static bool pf_gemm16()
{
    static const bool k16 = [] {
        const char* e = getenv("LG_PF_GEMM16");
        return e && e[0] == '1';
    }();
    return k16;
}

bool lg_prefill_gemm16() { return pf_gemm16(); }

/* the 32 x 32 product kernel (Q4_K, Q6_K): 128 rows x 64 tokens per
 * workgroup; two K halves in one workgroup where the tiles alone would give
 * one workgroup per CU or fewer (the 4096-row products at 512 tokens,
 * att_out and down: Q4_K 68.0 -> 61.8 us on average; Q|K|V's 384 tiles ran
 * faster unsplit, 48.7 against 55.2 us) */
template <int WT>
static int gemm_k32(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                    int accumulate, hipStream_t s)
{
    const int nrb = (rows + PF2_RB - 1) / PF2_RB + 7 & ~7;
    const int ntl = (T + 63) / 64;
    const bool ks2 = nrb * ntl <= 256 && cols >= 4 * 256;
    const dim3 grid((unsigned)(nrb * ntl)), blk(ks2 ? 2 * PF2_NT : PF2_NT);
#define PF2_LAUNCH(A, N) hipLaunchKernelGGL((k_pf_gemm_k32<WT, A, N>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo)
    if (accumulate) { if (ks2) PF2_LAUNCH(1, 2); else PF2_LAUNCH(1, 1); }
    else { if (ks2) PF2_LAUNCH(0, 2); else PF2_LAUNCH(0, 1); }
#undef PF2_LAUNCH
    return lg_check_launch("prefill gemm");
}

static int gemm_q4k(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                    int accumulate, hipStream_t s)
{
    if (!W || !out || rows <= 0 || cols <= 0 || cols % 256 || T <= 0 || T > x.tld || x.tld % 4 ||
        rsz != (uint32_t)(cols / 256) * LG_BS_Q4_K || ldo < rows) {
        lg_set_error("prefill gemm: bad arguments (rows %d, cols %d, T %d)", rows, cols, T);
        return LG_ERR_ARG;
    }
    if (!pf_gemm16()) return gemm_k32<LG_Q4_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    /* LG_PF_GEMM16=1: the 16 x 16 product kernel.  64-token tiles: 128
     * VGPRs, so up to four workgroups share a CU (at 128 tokens a workgroup
     * needs 220 and the 512-token up|gate GEMM ran 10% slower) */
    const int nrb8 = (rows + PF_RB - 1) / PF_RB + 7 & ~7;
#ifndef LG_PF_MI
#define LG_PF_MI 4
#endif
    const dim3 grid((unsigned)(nrb8 * ((T + 16 * LG_PF_MI - 1) / (16 * LG_PF_MI)))), blk(PF_NT);
    if (accumulate) hipLaunchKernelGGL((k_pf_gemm_q4k<1, LG_PF_MI>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    else hipLaunchKernelGGL((k_pf_gemm_q4k<0, LG_PF_MI>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    return lg_check_launch("prefill gemm");
}

int lg_prefill_quantize(int qtype, const float* x, int ldx, const float* norm_w, float eps, int n, int T,
                        const PfQ8K& q, hipStream_t s)
{
    if (!x || !(qtype == LG_F32 ? (void*)q.f : (void*)q.qs) || n <= 0 || n % (qtype == LG_Q8_K ? 256 : 32) ||
        T <= 0 || T > q.tld || ldx < n || (qtype != LG_Q8_K && qtype != LG_Q8_0 && qtype != LG_F32)) {
        lg_set_error("prefill quantize: bad arguments (type %d, n %d, T %d)", qtype, n, T);
        return LG_ERR_ARG;
    }
    const dim3 grid(T), blk(256);
    if (qtype == LG_Q8_K) hipLaunchKernelGGL(k_pf_quant<LG_Q8_K>, grid, blk, 0, s, x, ldx, norm_w, eps, n, q);
    else if (qtype == LG_Q8_0) hipLaunchKernelGGL(k_pf_quant<LG_Q8_0>, grid, blk, 0, s, x, ldx, norm_w, eps, n, q);
    else hipLaunchKernelGGL(k_pf_quant<LG_F32>, grid, blk, 0, s, x, ldx, norm_w, eps, n, q);
    return lg_check_launch("prefill quantize");
}

/* ------------------------------------------------------------------ */
/* Q1_G x Q8_0 GEMM on int8 MFMA                                        */
/* ------------------------------------------------------------------ */
/* A Q1_G block (18 B: fp16 d, 128 sign bits, bit i of byte i/8 = value i)
 * meets four Q8_0 activation blocks of 32.  dot_q8_0_q1_G
 * (fast/lil_math.cpp:440-464) takes per 32-value block the integer
 * 2 s1 - asum (s1 = sum of q where the bit is set, asum = sum of q) and
 * d_w * sum_j d_a,j (2 s1_j - asum_j).  Here s1 is one
 * v_mfma_i32_16x16x32_i8 per block with the bits as 0/1 bytes (K = 32: each
 * 32-value block has its own activation scale, so the products cannot run
 * over two blocks), asum comes with the activation, and
 * out += d_w * sum_j d_a,j (2 s1_j - asum_j) in fp32 per 128-value group.
 * Tile and staging as k_pf_gemm_q4k: 128 rows x 64 tokens per workgroup, 8
 * waves of 16 rows x 4 token tiles; per group the token tile's 128 quants
 * per token (rows padded to 144 B), the scales and asums in LDS,
 * double-buffered; lane group g takes values 8g..8g+7 of each block.  Up to
 * 256 VGPRs (one workgroup per CU): held to 128 the compiler spilled ~110. */
#define PF1_AST 144
template <int ACC>
__global__ __launch_bounds__(512) void k_pf_gemm_q1g(
    const uint8_t* __restrict__ W, uint32_t rsz, int R, int K, PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    constexpr int MI = 4;
    __shared__ __attribute__((aligned(16))) int8_t s_a[2][64 * PF1_AST];
    __shared__ __attribute__((aligned(16))) float s_d[2][4][64];
    __shared__ __attribute__((aligned(16))) int s_s[2][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int ng = K >> 7;
    const int nt = (T + 63) / 64;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * 128 >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * 64;
    const int r0 = rb * 128 + wave * 16;
    const uint8_t* wr = W + (size_t)min(r0 + l16, R - 1) * rsz;

    /* staging per group: thread tid takes 16 quants (token tid/8, piece
     * tid%8); threads < 64 four scales and four asums (block tid/16,
     * tokens 4(tid%16)..) */
    struct Stg {
        uint4 a;
        float4 d;
        int4 s;
    };
    auto stage_load = [&](Stg& st, int gi) {
        const int tok = min(t0 + (tid >> 3), T - 1);
        st.a = *(const uint4*)(x.qs + (size_t)tok * K + (size_t)gi * 128 + (tid & 7) * 16);
        const size_t di = (size_t)(4 * gi + ((tid >> 4) & 3)) * x.tld + min(t0 + 4 * (tid & 15), x.tld - 4);
        st.d = *(const float4*)(x.d + di);
        st.s = *(const int4*)(x.as + di);
    };
    auto stage_store = [&](const Stg& st, int buf) {
        *(uint4*)(s_a[buf] + (tid >> 3) * PF1_AST + (tid & 7) * 16) = st.a;
        if (tid < 64) {
            *(float4*)&s_d[buf][tid >> 4][4 * (tid & 15)] = st.d;
            *(int4*)&s_s[buf][tid >> 4][4 * (tid & 15)] = st.s;
        }
    };
    struct Blk {
        uint32_t d;
        uint4 bits;
    };
    auto blk_load = [&](Blk& B, int gi) {
        const uint8_t* p = wr + (size_t)gi * LG_BS_Q1_G;
        B.d = lg_ld16(p);
        B.bits = lg_ld<uint4>(p + 2);
    };

    v4f acc[MI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++) acc[mi] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int gi, const Blk& cur) {
        const int buf = gi & 1;
        const uint32_t bw[4] = {cur.bits.x, cur.bits.y, cur.bits.z, cur.bits.w};
        const float dw = lg_h2f((uint16_t)cur.d);
        v4f ga[MI];
#pragma unroll
        for (int mi = 0; mi < MI; mi++) ga[mi] = (v4f){0.f, 0.f, 0.f, 0.f};
        const int8_t* sa = s_a[buf] + l16 * PF1_AST + 8 * g;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            /* bits 32j + 8g.. = byte 4j + g of the 16 sign bytes */
            const uint32_t b8 = (bw[j] >> (8 * g)) & 0xFFu;
            const long bb = (long)((uint64_t)(uint32_t)bits4_to_bytes(b8 & 15u) |
                                   ((uint64_t)(uint32_t)bits4_to_bytes(b8 >> 4) << 32));
#pragma unroll
            for (int mi = 0; mi < MI; mi++) {
                const long af = *(const long*)(sa + 16 * mi * PF1_AST + 32 * j);
                const v4i s1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bb, (v4i){0, 0, 0, 0}, 0, 0, 0);
                const float4 da = *(const float4*)&s_d[buf][j][16 * mi + 4 * g];
                const int4 as = *(const int4*)&s_s[buf][j][16 * mi + 4 * g];
                const float dav[4] = {da.x, da.y, da.z, da.w};
                const int asv[4] = {as.x, as.y, as.z, as.w};
#pragma unroll
                for (int i = 0; i < 4; i++) ga[mi][i] = __builtin_fmaf(dav[i], (float)(2 * s1[i] - asv[i]), ga[mi][i]);
            }
        }
#pragma unroll
        for (int mi = 0; mi < MI; mi++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[mi][i] = __builtin_fmaf(dw, ga[mi][i], acc[mi][i]);
    };

    Blk cur, nxt;
    Stg st;
    stage_load(st, 0);
    blk_load(cur, 0);
    stage_store(st, 0);
    __syncthreads();
    for (int gi = 0; gi < ng; gi++) {
        const int gn = min(gi + 1, ng - 1);
        stage_load(st, gn);
        blk_load(nxt, gn);
        compute(gi, cur);
        stage_store(st, (gi + 1) & 1);
        cur = nxt;
        __syncthreads();
    }
    const int r = r0 + l16;
#pragma unroll
    for (int mi = 0; mi < MI; mi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * mi + 4 * g + i;
            if (t < T && r < R) {
                float* o = out + (size_t)t * ldo + r;
                *o = ACC ? *o + acc[mi][i] : acc[mi][i];
            }
        }
    }
}

static int gemm_q1g(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                    int accumulate, hipStream_t s)
{
    if (!W || !out || !x.as || rows <= 0 || cols <= 0 || cols % 256 || T <= 0 || T > x.tld || x.tld % 4 ||
        rsz != (uint32_t)(cols / 128) * LG_BS_Q1_G || ldo < rows) {
        lg_set_error("prefill gemm Q1_G: bad arguments (rows %d, cols %d, T %d)", rows, cols, T);
        return LG_ERR_ARG;
    }
    const int nrb8 = (rows + 127) / 128 + 7 & ~7;
    const dim3 grid((unsigned)(nrb8 * ((T + 63) / 64))), blk(512);
    if (accumulate) hipLaunchKernelGGL((k_pf_gemm_q1g<1>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    else hipLaunchKernelGGL((k_pf_gemm_q1g<0>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    return lg_check_launch("prefill gemm Q1_G");
}

/* ------------------------------------------------------------------ */
/* Q2_K, Q3_K, Q5_K, Q6_K x Q8_K GEMMs on int8 MFMA                      */
/* ------------------------------------------------------------------ */
/* Tile, grid and token staging as k_pf_gemm_q4k: 128 rows x 64 tokens per
 * workgroup, the Q8_K token tile of each 256-value block in LDS in the same
 * lane-group order (per 64-value chunk c, lane group g: the 8 values
 * 64c+8g.. then the 8 values 64c+32+8g..).  Each sub-block's integer sum
 * isum_j is one v_mfma_i32_16x16x32_i8 (8 bytes a lane): the first 8
 * staged bytes of every lane group are values 64c..64c+31, the second 8
 * values 64c+32..64c+63.  A 32-value sub-block (Q5_K) is one such product;
 * a 16-value one (Q2_K, Q3_K, Q6_K) is half of it, so two products run
 * with the weight bytes of lane groups 2,3 or 0,1 zeroed.  The sub-block
 * scale of the lane's row then multiplies isum_j in int32:
 * S = sum_j sc_j isum_j is the reference's integer (its aux32 / isum sums),
 * exact; the mins term M (Q2_K, Q5_K) is an fp32 MFMA product of the bsums
 * and the 4-bit / 6-bit mins, exact (integers below 2^24); per block
 *   Q2_K, Q5_K: out += d_a (d_w S - dmin_w M)
 *   Q3_K, Q6_K: out += (d_w d_a) S
 * fp32 rounding order aside, the reference's dot of each type. */
template <int WT>
struct PfKq;

/* Q2_K (84 B: scales[16], qs[64], d, dmin): value 128n + 32j + l is bits
 * 2j of qs[32n + l]; 16-value sub-block i: scale = low nibble of
 * scales[i], min = high nibble.  fast/lil_math.cpp:539-580 */
template <>
struct PfKq<LG_Q2_K> {
    static constexpr int SUB = 16, MINS = 1;
    struct Blk {
        uint2 q[2];
        uint4 sc;
        uint32_t dd;
    };
    static __device__ __forceinline__ void load(Blk& B, const uint8_t* p, int g)
    {
        B.q[0] = lg_ld<uint2>(p + 16 + 8 * g);
        B.q[1] = lg_ld<uint2>(p + 48 + 8 * g);
        B.sc = lg_ld<uint4>(p);
        B.dd = lg_ld<uint32_t>(p + 80);
    }
    /* the lane's 8 values of half h of chunk c (values 64c + 32h + 8g..) */
    static __device__ __forceinline__ uint2 vals(const Blk& B, int c, int h)
    {
        const int j = 2 * (c & 1) + h;
        const uint2 q = c >> 1 ? B.q[1] : B.q[0];
        return make_uint2((q.x >> (2 * j)) & 0x03030303u, (q.y >> (2 * j)) & 0x03030303u);
    }
    static __device__ __forceinline__ int scale(const Blk& B, int i) { return byte16(B.sc, i) & 15; }
    static __device__ __forceinline__ float minv(const Blk& B, int i) { return (float)(byte16(B.sc, i) >> 4); }
    static __device__ __forceinline__ float d(const Blk& B) { return lg_h2f((uint16_t)(B.dd & 0xffffu)); }
    static __device__ __forceinline__ float dmin(const Blk& B) { return lg_h2f((uint16_t)(B.dd >> 16)); }
};

/* Q3_K (110 B: hmask[32], qs[64], scales[12], d): value 128n + 32j + l is
 * bits 2j of qs[32n + l], minus 4 where bit 4n + j of hmask[l] is clear;
 * 16 six-bit scales minus 32.  fast/lil_math.cpp:466-537 */
template <>
struct PfKq<LG_Q3_K> {
    static constexpr int SUB = 16, MINS = 0;
    struct Blk {
        uint2 q[2], hm;
        uint32_t s0, s1, s2, d;
    };
    static __device__ __forceinline__ void load(Blk& B, const uint8_t* p, int g)
    {
        B.hm = lg_ld<uint2>(p + 8 * g);
        B.q[0] = lg_ld<uint2>(p + 32 + 8 * g);
        B.q[1] = lg_ld<uint2>(p + 64 + 8 * g);
        B.s0 = lg_ld<uint32_t>(p + 96);
        B.s1 = lg_ld<uint32_t>(p + 100);
        B.s2 = lg_ld<uint32_t>(p + 104);
        B.d = lg_ld16(p + 108);
    }
    static __device__ __forceinline__ uint2 vals(const Blk& B, int c, int h)
    {
        const int n = c >> 1, j = 2 * (c & 1) + h;
        const uint2 q = n ? B.q[1] : B.q[0];
        auto one = [&](uint32_t qw, uint32_t hw) {
            const uint32_t u = ((qw >> (2 * j)) & 0x03030303u) | (((hw >> (4 * n + j)) & 0x01010101u) << 2);
            return ((u | 0x80808080u) - 0x04040404u) ^ 0x80808080u;   /* bytewise u - 4 (u < 8) */
        };
        return make_uint2(one(q.x, B.hm.x), one(q.y, B.hm.y));
    }
    /* scale i: low nibble of byte i (i < 8) or high nibble of byte i - 8 of
     * the first 8 bytes, two high bits from byte 8 + (i & 3) at 2 (i / 4) */
    static __device__ __forceinline__ int scale(const Blk& B, int i)
    {
        const uint32_t lw = (i & 7) < 4 ? B.s0 : B.s1;
        const int lo = i < 8 ? byte_of(lw, i & 3) & 15 : byte_of(lw, i & 3) >> 4;
        const int hi = (byte_of(B.s2, i & 3) >> (2 * (i >> 2))) & 3;
        return (lo | (hi << 4)) - 32;
    }
    static __device__ __forceinline__ float minv(const Blk&, int) { return 0.0f; }
    static __device__ __forceinline__ float d(const Blk& B) { return lg_h2f((uint16_t)B.d); }
    static __device__ __forceinline__ float dmin(const Blk&) { return 0.0f; }
};

/* Q5_K (176 B: d, dmin, scales[12], qh[32], qs[128]): value 64c + 32h + i
 * is nibble h of qs[32c + i] plus 16 x bit 2c + h of qh[i]; 32-value
 * sub-blocks with the Q4_K scale/min packing.  fast/lil_math.cpp:618-686 */
template <>
struct PfKq<LG_Q5_K> {
    static constexpr int SUB = 32, MINS = 1;
    struct Blk {
        uint4 hdr;
        uint2 qh, q[4];
    };
    static __device__ __forceinline__ void load(Blk& B, const uint8_t* p, int g)
    {
        B.hdr = lg_ld<uint4>(p);
        B.qh = lg_ld<uint2>(p + 16 + 8 * g);
#pragma unroll
        for (int c = 0; c < 4; c++) B.q[c] = lg_ld<uint2>(p + 48 + 32 * c + 8 * g);
    }
    static __device__ __forceinline__ uint2 vals(const Blk& B, int c, int h)
    {
        auto one = [&](uint32_t qw, uint32_t hw) {
            return ((qw >> (4 * h)) & 0x0F0F0F0Fu) | (((hw >> (2 * c + h)) & 0x01010101u) << 4);
        };
        const uint2 q = c == 0 ? B.q[0] : c == 1 ? B.q[1] : c == 2 ? B.q[2] : B.q[3];
        return make_uint2(one(q.x, B.qh.x), one(q.y, B.qh.y));
    }
    /* get_scale_min_k4 (fast/lil_math.cpp:129-138) */
    static __device__ __forceinline__ int scale(const Blk& B, int j)
    {
        const uint32_t w = j < 4 ? B.hdr.y & 0x3F3F3F3Fu : (B.hdr.w & 0x0F0F0F0Fu) | ((B.hdr.y >> 2) & 0x30303030u);
        return byte_of(w, j & 3);
    }
    static __device__ __forceinline__ float minv(const Blk& B, int j)
    {
        const uint32_t w = j < 4 ? B.hdr.z & 0x3F3F3F3Fu
                                 : ((B.hdr.w >> 4) & 0x0F0F0F0Fu) | ((B.hdr.z >> 2) & 0x30303030u);
        return (float)byte_of(w, j & 3);
    }
    static __device__ __forceinline__ float d(const Blk& B) { return lg_h2f((uint16_t)(B.hdr.x & 0xffffu)); }
    static __device__ __forceinline__ float dmin(const Blk& B) { return lg_h2f((uint16_t)(B.hdr.x >> 16)); }
};

/* Q6_K (210 B: ql[128], qh[64], scales[16] int8, d): value
 * 128n + 64c' + 32h + l is nibble c' of ql[64n + 32h + l] with bits
 * 2(2c' + h) of qh[32n + l] above it, minus 32.  fast/lil_math.cpp:688-739 */
template <>
struct PfKq<LG_Q6_K> {
    static constexpr int SUB = 16, MINS = 0;
    struct Blk {
        uint2 ql[2][2], qh[2];
        uint4 sc;
        uint32_t d;
    };
    static __device__ __forceinline__ void load(Blk& B, const uint8_t* p, int g)
    {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            B.ql[n][0] = lg_ld<uint2>(p + 64 * n + 8 * g);
            B.ql[n][1] = lg_ld<uint2>(p + 64 * n + 32 + 8 * g);
            B.qh[n] = lg_ld<uint2>(p + 128 + 32 * n + 8 * g);
        }
        B.sc = lg_ld<uint4>(p + 192);
        B.d = lg_ld16(p + 208);
    }
    static __device__ __forceinline__ uint2 vals(const Blk& B, int c, int h)
    {
        const int n = c >> 1, cp = c & 1, sh = 2 * (2 * cp + h);
        const uint2 l = n ? B.ql[1][h] : B.ql[0][h], hq = n ? B.qh[1] : B.qh[0];
        auto one = [&](uint32_t lw, uint32_t hw) {
            const uint32_t u = ((lw >> (4 * cp)) & 0x0F0F0F0Fu) | (((hw >> sh) & 0x03030303u) << 4);
            return ((u | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   /* bytewise u - 32 (u < 64) */
        };
        return make_uint2(one(l.x, hq.x), one(l.y, hq.y));
    }
    static __device__ __forceinline__ int scale(const Blk& B, int i) { return (int)(int8_t)byte16(B.sc, i); }
    static __device__ __forceinline__ float minv(const Blk&, int) { return 0.0f; }
    static __device__ __forceinline__ float d(const Blk& B) { return lg_h2f((uint16_t)B.d); }
    static __device__ __forceinline__ float dmin(const Blk&) { return 0.0f; }
};

__device__ __forceinline__ long pf_u2l(uint2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }

template <int WT, int ACC>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gemm_kq(
    const uint8_t* __restrict__ W, uint32_t rsz, int R, int K, PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    using F = PfKq<WT>;
    constexpr int MI = 4, BSZ = WT == LG_Q2_K ? LG_BS_Q2_K : WT == LG_Q3_K ? LG_BS_Q3_K : WT == LG_Q5_K ? LG_BS_Q5_K : LG_BS_Q6_K;
    __shared__ __attribute__((aligned(16))) int8_t s_a[2][64 * PF_AST];
    __shared__ __attribute__((aligned(16))) int16_t s_bs[2][64 * 16];
    __shared__ __attribute__((aligned(16))) float s_d[2][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int nb = K >> 8;
    const int nt = (T + 63) / 64;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * 128 >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * 64;
    const int r0 = rb * 128 + wave * 16;
    const uint8_t* wr = W + (size_t)min(r0 + l16, R - 1) * rsz;

    /* staging per block as k_pf_gemm_q4k with 64 tokens: thread tid takes
     * quant chunks tid and tid + 512 (token chunk/16, 16-byte piece
     * chunk%16), a quarter of token tid/4's bsums (tid < 256) and four block
     * scales (tid < 16) */
    struct Stg {
        uint4 a[2];
        uint2 bs;
        uint4 d;
    };
    auto stage_load = [&](Stg& st, int b) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = tid + 512 * i, tok = min(t0 + (q >> 4), T - 1);
            st.a[i] = *(const uint4*)(x.qs + (size_t)tok * K + (size_t)b * 256 + (q & 15) * 16);
        }
        const int tb = min(t0 + ((tid >> 2) & 63), T - 1);
        st.bs = *(const uint2*)(x.bs + ((size_t)tb * nb + b) * 16 + (tid & 3) * 4);
        st.d = *(const uint4*)(x.d + (size_t)b * x.tld + min(t0 + 4 * (tid & 15), x.tld - 4));
    };
    auto stage_store = [&](const Stg& st, int buf) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = tid + 512 * i, p = q & 15, k = p & 3;
            int8_t* dst = s_a[buf] + (q >> 4) * PF_AST + 64 * (p >> 2) + 32 * (k & 1) + 8 * (k >> 1);
            *(uint2*)dst = make_uint2(st.a[i].x, st.a[i].y);
            *(uint2*)(dst + 16) = make_uint2(st.a[i].z, st.a[i].w);
        }
        if (tid < 256) *(uint2*)(s_bs[buf] + (tid >> 2) * 16 + (tid & 3) * 4) = st.bs;
        if (tid < 16) *(uint4*)(s_d[buf] + 4 * tid) = st.d;
    };

    v4f acc[MI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++) acc[mi] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int b, const typename F::Blk& cur) {
        const int buf = b & 1;
        v4i S[MI];
#pragma unroll
        for (int mi = 0; mi < MI; mi++) S[mi] = (v4i){0, 0, 0, 0};
        const int8_t* sa = s_a[buf] + l16 * PF_AST + 16 * g;
        /* one chunk at a time for the 16-value types: the 16 products of a
         * chunk give the MFMA enough independent work, and more chunks in
         * flight spill */
        constexpr int UC = F::SUB == 16 ? 1 : 4;
#pragma unroll UC
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const long bw = pf_u2l(F::vals(cur, c, h));
                if constexpr (F::SUB == 32) {
                    const int sc = F::scale(cur, 2 * c + h);
#pragma unroll
                    for (int mi = 0; mi < MI; mi++) {
                        const long a = *(const long*)(sa + 16 * mi * PF_AST + 64 * c + 8 * h);
                        const v4i is = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bw, (v4i){0, 0, 0, 0}, 0, 0, 0);
                        S[mi] += sc * is;
                    }
                } else {
                    /* sub-blocks 4c + 2h (lane groups 0, 1) and 4c + 2h + 1 (groups 2, 3) */
                    const long b0 = g < 2 ? bw : 0L, b1 = g < 2 ? 0L : bw;
                    const int sc0 = F::scale(cur, 4 * c + 2 * h), sc1 = F::scale(cur, 4 * c + 2 * h + 1);
#pragma unroll
                    for (int mi = 0; mi < MI; mi++) {
                        const long a = *(const long*)(sa + 16 * mi * PF_AST + 64 * c + 8 * h);
                        const v4i i0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, (v4i){0, 0, 0, 0}, 0, 0, 0);
                        const v4i i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, (v4i){0, 0, 0, 0}, 0, 0, 0);
                        S[mi] += sc0 * i0 + sc1 * i1;
                    }
                }
            }
        }
        const float dw = F::d(cur), dmw = F::dmin(cur);
#pragma unroll
        for (int mi = 0; mi < MI; mi++) {
            const float4 dx = *(const float4*)(s_d[buf] + 16 * mi + 4 * g);
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
            if constexpr (F::MINS) {
                /* M[token][row] = sum_i min_i bsum_i (k = g: the lane's mins) */
                const int16_t* bsr = s_bs[buf] + (16 * mi + l16) * 16;
                v4f M = (v4f){0.f, 0.f, 0.f, 0.f};
                if constexpr (F::SUB == 16) {
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        M = __builtin_amdgcn_mfma_f32_16x16x4f32((float)bsr[4 * q + g], F::minv(cur, 4 * q + g), M, 0, 0, 0);
                } else {
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int j = 4 * q + g, v = *(const int*)(bsr + 2 * j);
                        const float bp = (float)((int)(int16_t)(v & 0xffff) + (int)(int16_t)(v >> 16));
                        M = __builtin_amdgcn_mfma_f32_16x16x4f32(bp, F::minv(cur, j), M, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[mi][i] = __builtin_fmaf(dxs[i], lg_fma2(dw, (float)S[mi][i], -dmw, M[i]), acc[mi][i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mi][i] = __builtin_fmaf(dw * dxs[i], (float)S[mi][i], acc[mi][i]);
            }
        }
    };

    typename F::Blk cur, nxt;
    Stg st;
    stage_load(st, 0);
    F::load(cur, wr, g);
    stage_store(st, 0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int bn = min(b + 1, nb - 1);
        stage_load(st, bn);
        F::load(nxt, wr + (size_t)bn * BSZ, g);
        compute(b, cur);
        stage_store(st, (b + 1) & 1);
        cur = nxt;
        __syncthreads();
    }
    const int r = r0 + l16;
#pragma unroll
    for (int mi = 0; mi < MI; mi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * mi + 4 * g + i;
            if (t < T && r < R) {
                float* o = out + (size_t)t * ldo + r;
                *o = ACC ? *o + acc[mi][i] : acc[mi][i];
            }
        }
    }
}

template <int WT>
static int gemm_kq(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                   int accumulate, hipStream_t s)
{
    const int nrb8 = (rows + 127) / 128 + 7 & ~7;
    const dim3 grid((unsigned)(nrb8 * ((T + 63) / 64))), blk(512);
    if (accumulate) hipLaunchKernelGGL((k_pf_gemm_kq<WT, 1>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    else hipLaunchKernelGGL((k_pf_gemm_kq<WT, 0>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    return lg_check_launch("prefill gemm (K-quant)");
}

/* ------------------------------------------------------------------ */
/* Q8_0 and Q1_0 x Q8_0 GEMMs on int8 MFMA                              */
/* ------------------------------------------------------------------ */
/* dot_q8_0_q8_0 and dot_q8_0_q1_0 (fast/lil_math.cpp:411-438): per 32-value
 * block the integer sum s of w*q (Q1_0: w = +1 where the bit is set, else
 * -1), then acc += d_w d_a s.  s is one v_mfma_i32_16x16x32_i8 (lane group
 * g feeds values 8g..8g+7 of the block: 8 Q8_0 bytes, or bit byte g of a
 * Q1_0 block as +-1 bytes), exact; the fp32 combination runs per block.
 * Tile and staging as k_pf_gemm_q1g: 128 rows x 64 tokens, the token
 * tile's quants in groups of 4 blocks (128 values) in LDS with their
 * scales, double-buffered.  The width need only be a multiple of 32: a
 * last group of fewer than 4 blocks stages clamped bytes it never uses. */
/* where block `blk` of a row keeps its d and its quants (Q8_0) or sign
 * bits (Q1_0): GGUF blocks, or the regrouped rows of the fused decode step
 * (LG_Q8_0_R / LG_Q1_0_R: per run of 8 blocks, the 8 blocks' quants or
 * bits, then their 8 d) */
template <int WT>
struct PfB32 {
    static constexpr bool Q8 = WT == LG_Q8_0 || WT == LG_Q8_0_R;
    static constexpr bool REP = WT == LG_Q8_0_R || WT == LG_Q1_0_R;
    static constexpr int BSZ = Q8 ? LG_BS_Q8_0 : LG_BS_Q1_0;
    static constexpr int QB = Q8 ? 32 : 4;   /* quant / bit bytes per block */
    static __device__ __forceinline__ const uint8_t* d(const uint8_t* row, int blk)
    {
        return REP ? row + (size_t)(blk >> 3) * 8 * BSZ + 8 * QB + 2 * (blk & 7) : row + (size_t)blk * BSZ;
    }
    static __device__ __forceinline__ const uint8_t* q(const uint8_t* row, int blk)
    {
        return REP ? row + (size_t)(blk >> 3) * 8 * BSZ + QB * (blk & 7) : row + (size_t)blk * BSZ + 2;
    }
};

template <int WT, int ACC>
__global__ __launch_bounds__(512) void k_pf_gemm_b32(
    const uint8_t* __restrict__ W, uint32_t rsz, int R, int K, PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    using B32 = PfB32<WT>;
    constexpr int MI = 4;
    __shared__ __attribute__((aligned(16))) int8_t s_a[2][64 * PF1_AST];
    __shared__ __attribute__((aligned(16))) float s_d[2][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int nbk = K >> 5, ng = (nbk + 3) >> 2;
    const int nt = (T + 63) / 64;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * 128 >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * 64;
    const int r0 = rb * 128 + wave * 16;
    const uint8_t* wr = W + (size_t)min(r0 + l16, R - 1) * rsz;

    struct Stg {
        uint4 a;
        float4 d;
    };
    auto stage_load = [&](Stg& st, int gi) {
        const int tok = min(t0 + (tid >> 3), T - 1);
        st.a = *(const uint4*)(x.qs + (size_t)tok * K + min(gi * 128 + (tid & 7) * 16, K - 16));
        const size_t di = (size_t)min(4 * gi + ((tid >> 4) & 3), nbk - 1) * x.tld + min(t0 + 4 * (tid & 15), x.tld - 4);
        st.d = *(const float4*)(x.d + di);
    };
    auto stage_store = [&](const Stg& st, int buf) {
        *(uint4*)(s_a[buf] + (tid >> 3) * PF1_AST + (tid & 7) * 16) = st.a;
        if (tid < 64) *(float4*)&s_d[buf][tid >> 4][4 * (tid & 15)] = st.d;
    };
    struct Blk {
        uint32_t d[4];
        uint2 q[4];
    };
    auto blk_load = [&](Blk& B, int gi) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int bk = min(4 * gi + j, nbk - 1);
            B.d[j] = lg_ld16(B32::d(wr, bk));
            if constexpr (B32::Q8) {
                B.q[j] = lg_ld<uint2>(B32::q(wr, bk) + 8 * g);
            } else {
                const uint32_t b8 = B32::q(wr, bk)[g];
                /* bit i -> byte i: +1 where set, -1 (0xFF) where clear */
                B.q[j] = make_uint2(0xFFFFFFFFu ^ ((uint32_t)bits4_to_bytes(b8 & 15u) * 0xFEu),
                                    0xFFFFFFFFu ^ ((uint32_t)bits4_to_bytes(b8 >> 4) * 0xFEu));
            }
        }
    };

    v4f acc[MI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++) acc[mi] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int gi, const Blk& cur) {
        const int buf = gi & 1;
        const int8_t* sa = s_a[buf] + l16 * PF1_AST + 8 * g;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (4 * gi + j >= nbk) break;   /* the last group's missing blocks (uniform) */
            const long bw = pf_u2l(cur.q[j]);
            const float dw = lg_h2f((uint16_t)cur.d[j]);
#pragma unroll
            for (int mi = 0; mi < MI; mi++) {
                const long a = *(const long*)(sa + 16 * mi * PF1_AST + 32 * j);
                const v4i is = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bw, (v4i){0, 0, 0, 0}, 0, 0, 0);
                const float4 da = *(const float4*)&s_d[buf][j][16 * mi + 4 * g];
                const float dav[4] = {da.x, da.y, da.z, da.w};
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mi][i] = __builtin_fmaf(dw * dav[i], (float)is[i], acc[mi][i]);
            }
        }
    };

    Blk cur, nxt;
    Stg st;
    stage_load(st, 0);
    blk_load(cur, 0);
    stage_store(st, 0);
    __syncthreads();
    for (int gi = 0; gi < ng; gi++) {
        const int gn = min(gi + 1, ng - 1);
        stage_load(st, gn);
        blk_load(nxt, gn);
        compute(gi, cur);
        stage_store(st, (gi + 1) & 1);
        cur = nxt;
        __syncthreads();
    }
    const int r = r0 + l16;
#pragma unroll
    for (int mi = 0; mi < MI; mi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * mi + 4 * g + i;
            if (t < T && r < R) {
                float* o = out + (size_t)t * ldo + r;
                *o = ACC ? *o + acc[mi][i] : acc[mi][i];
            }
        }
    }
}

/* The same products on the 32 x 32 forms (k_pf_gemm_k32's tile: 128 rows
 * x 64 tokens per workgroup of 4 waves, a wave 32 rows x two 32-token C
 * tiles, the token tile of 8 blocks (256 values) a step staged two steps
 * ahead, K in two halves where the tiles alone would leave one workgroup
 * per CU).  Per 32-value block: the integer sum is one
 * v_mfma_i32_32x32x32_i8 (lane l: row l % 32's bytes 16 (l / 32) .. +15 of
 * the block -- Q8_0 quants, or Q1_0 bits as +-1 bytes -- against the
 * token's), and the scale d_w d_a of every (token, row) pair of the tile is
 * one v_mfma_f32_32x32x16_f16 whose only nonzero K term is d_a (the
 * token's, fp16 as quantized) times d_w (the row's fp16): exact, and laid
 * out as the sums are, so each pair takes one convert and one fma, with no
 * per-token scale read from LDS.  out += (d_w d_a) s as k_pf_gemm_b32
 * (the same bits where K is not split).  Widths any multiple of 32: blocks
 * past the last of a step are not computed (their staged bytes are clamped
 * copies).
 *
 * Q1_G rows (WT = LG_Q1_G, LG_Q1_G_R): a 128-value block of sign bits with
 * one fp16 d_w meets four activation blocks; with the bits as +-1 bytes s is
 * dot_q8_0_q1_G's 2 s1 - asum, the scale MFMA puts d_a alone in place (B =
 * 1), and out += d_w sum_j d_a,j s_j per 128 values in k_pf_gemm_q1g's fp32
 * operations (the same bits where K is not split). */
template <int WT, int ACC, int KS>
__global__ __launch_bounds__(PF2_NT * KS) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gemm_b32x(
    const uint8_t* __restrict__ W, uint32_t rsz, int R, int K, PfQ8K x, int T, float* __restrict__ out, int ldo)
{
    constexpr bool G = WT == LG_Q1_G || WT == LG_Q1_G_R;   /* 128-value sign blocks */
    using B32 = PfB32<G ? LG_Q1_0 : WT>;
    constexpr int TT = 64;
    __shared__ __attribute__((aligned(16))) int8_t s_a[KS][2][TT * PF2_AST];
    __shared__ __attribute__((aligned(16))) _Float16 s_d[KS][2][8][TT];   /* d_a per block of the step, per token */
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kh = wave >> 2, tid = threadIdx.x & (PF2_NT - 1);
    const int h = lane >> 5, j = lane & 31;
    const int nbk = K >> 5, nst = (nbk + 7) >> 3;
    const int ns0 = KS == 2 ? (nst + 1) / 2 : nst;
    const int s0 = kh * ns0, nsh = kh ? nst - ns0 : ns0, L = ns0;
    const int nt = (T + TT - 1) / TT;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rb = (slot / nt) * 8 + xcd;
    if (rb * PF2_RB >= R) return;   /* padding of the row blocks to a multiple of 8 (whole workgroup) */
    const int t0 = (slot % nt) * TT;
    const int row = rb * PF2_RB + (wave & 3) * 32 + j;
    const uint8_t* wr = W + (size_t)min(row, R - 1) * rsz;
    int8_t(*sa_)[TT * PF2_AST] = s_a[kh];
    _Float16(*sd_)[8][TT] = s_d[kh];

    /* staging, per step: quant piece q = tid + 256 u (token q / 16, 16-byte
     * piece q % 16 of the step's 256 values, clamped to the row's end), and
     * d_a of blocks tid / 64 and tid / 64 + 4 of token tid % 64 */
    struct Stg {
        v4i a[4];
        float d[2];
    };
    auto stage_load = [&](Stg& st, int sp) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = tid + PF2_NT * u, tok = min(t0 + (q >> 4), T - 1);
            st.a[u] = *(const v4i*)(x.qs + (size_t)tok * K + min(sp * 256 + (q & 15) * 16, K - 16));
        }
        const int tok = min(t0 + (tid & 63), T - 1);
#pragma unroll
        for (int e = 0; e < 2; e++) st.d[e] = x.d[(size_t)min(8 * sp + (tid >> 6) + 4 * e, nbk - 1) * x.tld + tok];
    };
    auto stage_store = [&](const Stg& st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = tid + PF2_NT * u;
            *(v4i*)(sa_[buf] + (q >> 4) * PF2_AST + (q & 15) * 16) = st.a[u];
        }
#pragma unroll
        for (int e = 0; e < 2; e++) sd_[buf][(tid >> 6) + 4 * e][tid & 63] = (_Float16)st.d[e];
    };
    /* the lane's bytes of the step's 8 blocks and their d_w */
    struct Blk {
        v4i q[8];
        uint32_t d[4];
    };
    auto blk_load = [&](Blk& B, int sp) __attribute__((always_inline)) {
        if constexpr (G) {
            /* the step's two Q1_G blocks 2 sp, 2 sp + 1 (K is a multiple of 256):
             * bits 32 (e % 4) + 16h .. of block e / 4, and the two d_w */
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int qb = 2 * sp + (e >> 2);
                const uint8_t* bits = WT == LG_Q1_G_R ? wr + (size_t)(qb >> 3) * 8 * LG_BS_Q1_G + 16 * (qb & 7)
                                                      : wr + (size_t)qb * LG_BS_Q1_G + 2;
                const uint32_t b16 = lg_ld16(bits + 4 * (e & 3) + 2 * h);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    B.q[e][k] = (int)(0xFFFFFFFFu ^ ((uint32_t)bits4_to_bytes((b16 >> (4 * k)) & 15u) * 0xFEu));
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int qb = 2 * sp + u;
                B.d[u] = lg_ld16(WT == LG_Q1_G_R ? wr + (size_t)(qb >> 3) * 8 * LG_BS_Q1_G + 128 + 2 * (qb & 7)
                                                 : wr + (size_t)qb * LG_BS_Q1_G);
            }
        } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int bk = min(8 * sp + e, nbk - 1);
            if constexpr (B32::Q8) {
                B.q[e] = lg_ld<v4i>(B32::q(wr, bk) + 16 * h);   /* 16-byte aligned when regrouped */
            } else {
                /* bits 16h .. 16h + 15: bit i -> byte i, +1 where set, -1 where clear */
                const uint32_t b16 = lg_ld16(B32::q(wr, bk) + 2 * h);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    B.q[e][k] = (int)(0xFFFFFFFFu ^ ((uint32_t)bits4_to_bytes((b16 >> (4 * k)) & 15u) * 0xFEu));
            }
            if constexpr (!B32::REP) {
                const uint32_t dh = lg_ld16(B32::d(wr, bk));
                B.d[e >> 1] = (e & 1) ? (B.d[e >> 1] | (dh << 16)) : dh;
            }
        }
        if constexpr (B32::REP) {
            /* the step is one regrouped run: its 8 d in one load */
            const v4i dd = *(const v4i*)B32::d(wr, 8 * sp);
#pragma unroll
            for (int k = 0; k < 4; k++) B.d[k] = (uint32_t)dd[k];
        }
        }
    };

    v16f acc[2];
    acc[0] = (v16f){};
    acc[1] = (v16f){};

    auto compute = [&](int buf, const Blk& cur, int sp) __attribute__((always_inline)) {
        const int8_t* sa = sa_[buf] + j * PF2_AST + 16 * h;
        if constexpr (G) {
            v8h one = (v8h){};
            one[0] = h ? (_Float16)0.0f : (_Float16)1.0f;
            /* per Q1_G block u and tile t: g = sum_j d_a,j s_j over its four
             * activation blocks, then acc += d_w g */
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float dw = lg_h2f((uint16_t)cur.d[u]);
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    v16f g = (v16f){};
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int e = 4 * u + jj;
                        /* never taken (K is a multiple of 256), but a branch per
                         * block keeps the compiler from hoisting every block's
                         * products at once: fully unrolled, they spilled */
                        if (8 * sp + e >= nbk) break;
                        const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * e);
                        const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                        const v16i is = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, cur.q[e], (v16i){}, 0, 0, 0);
                        v8h ad = (v8h){};
                        ad[0] = h ? (_Float16)0.0f : sd_[buf][e][32 * t + j];
                        const v16f da = __builtin_amdgcn_mfma_f32_32x32x16_f16(ad, one, (v16f){}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) g[r] = __builtin_fmaf(da[r], (float)is[r], g[r]);
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[t][r] = __builtin_fmaf(dw, g[r], acc[t][r]);
                }
            }
        } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (8 * sp + e >= nbk) break;   /* past the last block (uniform) */
            /* scale operands: K term 0 only (lanes 0..31) */
            v8h bd = (v8h){};
            bd[0] = h ? (_Float16)0.0f : __builtin_bit_cast(_Float16, (uint16_t)(cur.d[e >> 1] >> (16 * (e & 1))));
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 a = *(const uint4*)(sa + 32 * t * PF2_AST + 32 * e);
                const v4i af = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                const v16i is = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, cur.q[e], (v16i){}, 0, 0, 0);
                v8h ad = (v8h){};
                ad[0] = h ? (_Float16)0.0f : sd_[buf][e][32 * t + j];
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ad, bd, (v16f){}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] = __builtin_fmaf(sc[r], (float)is[r], acc[t][r]);
            }
        }
        }
    };

    auto stp = [&](int i) { return s0 + min(i, nsh - 1); };
    Blk cur, nxt;
    Stg st0, st1;
    stage_load(st0, stp(0));
    stage_load(st1, stp(1));
    blk_load(cur, stp(0));
    stage_store(st0, 0);
    __syncthreads();
#define PF3_STEP(ii, ST_LD, ST_ST)                           \
    do {                                                     \
        stage_load(ST_LD, stp((ii) + 2));                    \
        blk_load(nxt, stp((ii) + 1));                        \
        if ((ii) < nsh) compute((ii) & 1, cur, s0 + (ii));   \
        stage_store(ST_ST, ((ii) + 1) & 1);                  \
        cur = nxt;                                           \
        __syncthreads();                                     \
    } while (0)
    for (int i = 0; i < L; i += 2) {
        PF3_STEP(i, st0, st1);
        PF3_STEP(i + 1, st1, st0);
    }
#undef PF3_STEP
    if constexpr (KS == 2) {
        float* red = (float*)s_a[1];
        if (kh == 1) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[(t * 16 + r) * (PF2_NT) + tid] = acc[t][r];
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][r] = acc[t][r] + red[(t * 16 + r) * (PF2_NT) + tid];
    }
    if (row < R) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int tok = t0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                if (tok < T) {
                    float* o = out + (size_t)tok * ldo + row;
                    *o = ACC ? *o + acc[t][r] : acc[t][r];
                }
            }
        }
    }
}

template <int WT>
static int gemm_b32x(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                     int accumulate, hipStream_t s)
{
    const int nrb = (rows + PF2_RB - 1) / PF2_RB + 7 & ~7;
    const int ntl = (T + 63) / 64;
    const bool ks2 = nrb * ntl <= 256 && cols >= 4 * 256;
    const dim3 grid((unsigned)(nrb * ntl)), blk(ks2 ? 2 * PF2_NT : PF2_NT);
#define PF3_LAUNCH(A, N) hipLaunchKernelGGL((k_pf_gemm_b32x<WT, A, N>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo)
    if (accumulate) { if (ks2) PF3_LAUNCH(1, 2); else PF3_LAUNCH(1, 1); }
    else { if (ks2) PF3_LAUNCH(0, 2); else PF3_LAUNCH(0, 1); }
#undef PF3_LAUNCH
    return lg_check_launch("prefill gemm (32-value blocks)");
}

template <int WT>
static int gemm_b32(const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out, int ldo,
                    int accumulate, hipStream_t s)
{
    if (!pf_gemm16()) return gemm_b32x<WT>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    const int nrb8 = (rows + 127) / 128 + 7 & ~7;
    const dim3 grid((unsigned)(nrb8 * ((T + 63) / 64))), blk(512);
    if (accumulate) hipLaunchKernelGGL((k_pf_gemm_b32<WT, 1>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    else hipLaunchKernelGGL((k_pf_gemm_b32<WT, 0>), grid, blk, 0, s, W, rsz, rows, cols, x, T, out, ldo);
    return lg_check_launch("prefill gemm (32-value blocks)");
}

int lg_prefill_act_type(int wtype)
{
    switch (wtype) {
    case LG_Q2_K: case LG_Q3_K: case LG_Q4_K: case LG_Q5_K: case LG_Q6_K: case LG_Q6_K_R: return LG_Q8_K;
    case LG_Q8_0: case LG_Q1_0: case LG_Q1_G: case LG_Q8_0_R: case LG_Q1_0_R: case LG_Q1_G_R: return LG_Q8_0;
    case LG_F32: case LG_F16: return LG_F32;
    default: return -1;
    }
}

static int64_t pf_row_bytes(int wtype, int cols)
{
    switch (wtype) {
    case LG_Q2_K: return cols % 256 ? -1 : (int64_t)cols / 256 * LG_BS_Q2_K;
    case LG_Q3_K: return cols % 256 ? -1 : (int64_t)cols / 256 * LG_BS_Q3_K;
    case LG_Q4_K: return cols % 256 ? -1 : (int64_t)cols / 256 * LG_BS_Q4_K;
    case LG_Q5_K: return cols % 256 ? -1 : (int64_t)cols / 256 * LG_BS_Q5_K;
    case LG_Q6_K: return cols % 256 ? -1 : (int64_t)cols / 256 * LG_BS_Q6_K;
    case LG_Q6_K_R: return cols % 2048 ? -1 : (int64_t)cols / 256 * LG_BS_Q6_K;
    case LG_Q8_0: return cols % 32 ? -1 : (int64_t)cols / 32 * LG_BS_Q8_0;
    case LG_Q1_0: return cols % 32 ? -1 : (int64_t)cols / 32 * LG_BS_Q1_0;
    /* regrouped rows: whole runs of 8 blocks */
    case LG_Q8_0_R: return cols % 256 ? -1 : (int64_t)cols / 32 * LG_BS_Q8_0;
    case LG_Q1_0_R: return cols % 256 ? -1 : (int64_t)cols / 32 * LG_BS_Q1_0;
    case LG_Q1_G: return cols % 256 ? -1 : (int64_t)cols / 128 * LG_BS_Q1_G;   /* the Q1_G GEMM steps 256 values */
    case LG_Q1_G_R: return cols % 1024 ? -1 : (int64_t)cols / 128 * LG_BS_Q1_G;
    case LG_F32: return cols % 32 ? -1 : (int64_t)cols * 4;
    case LG_F16: return cols % 32 ? -1 : (int64_t)cols * 2;
    default: return -1;
    }
}

int lg_prefill_gemm(int wtype, const uint8_t* W, uint32_t rsz, int rows, int cols, const PfQ8K& x, int T, float* out,
                    int ldo, int accumulate, hipStream_t s)
{
    const int at = lg_prefill_act_type(wtype);
    if (at < 0) {
        lg_set_error("prefill gemm: weight type %d is not batched", wtype);
        return LG_ERR_TYPE;
    }
    const int64_t rb = pf_row_bytes(wtype, cols);
    if (at == LG_F32) {
        if (rb < 0 || rsz != (uint32_t)rb || !x.f || T > x.tld) {
            lg_set_error("prefill gemm: bad arguments (type %d, cols %d, row bytes %u, T %d)", wtype, cols, rsz, T);
            return LG_ERR_ARG;
        }
        return lg_fgemm_tokens(wtype, W, rows, cols, x.f, cols, T, out, ldo, accumulate, s);
    }
    if (!W || !out || !x.qs || !x.d || (at == LG_Q8_K && !x.bs) || (wtype == LG_Q1_G && !x.as) || rows <= 0 ||
        cols < 32 || rb < 0 || rsz != (uint32_t)rb || T <= 0 || T > x.tld || x.tld % 4 || ldo < rows) {
        lg_set_error("prefill gemm: bad arguments (type %d, rows %d, cols %d, row bytes %u, T %d)", wtype, rows, cols,
                     rsz, T);
        return LG_ERR_ARG;
    }
    switch (wtype) {
    case LG_Q4_K: return gemm_q4k(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q1_G:
        if (!pf_gemm16()) return gemm_b32x<LG_Q1_G>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
        return gemm_q1g(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q1_G_R:
        if (pf_gemm16()) {
            lg_set_error("prefill gemm: regrouped Q1_G rows take the 32 x 32 kernel");
            return LG_ERR_ARG;
        }
        return gemm_b32x<LG_Q1_G_R>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q2_K:
        if (!pf_gemm16()) return gemm_k32<LG_Q2_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
        return gemm_kq<LG_Q2_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q3_K:
        if (!pf_gemm16()) return gemm_k32<LG_Q3_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
        return gemm_kq<LG_Q3_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q5_K:
        if (!pf_gemm16()) return gemm_k32<LG_Q5_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
        return gemm_kq<LG_Q5_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q6_K:
        if (!pf_gemm16()) return gemm_k32<LG_Q6_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
        return gemm_kq<LG_Q6_K>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q6_K_R:
        if (pf_gemm16()) {
            lg_set_error("prefill gemm: regrouped Q6_K rows take the 32 x 32 kernel");
            return LG_ERR_ARG;
        }
        return gemm_k32<LG_Q6_K_R>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q8_0: return gemm_b32<LG_Q8_0>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q8_0_R: return gemm_b32<LG_Q8_0_R>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    case LG_Q1_0_R: return gemm_b32<LG_Q1_0_R>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    default: return gemm_b32<LG_Q1_0>(W, rsz, rows, cols, x, T, out, ldo, accumulate, s);
    }
}

/* ------------------------------------------------------------------ */
/* causal attention on fp16 MFMA: 16 query tokens x one KV head          */
/* ------------------------------------------------------------------ */
/* One workgroup per (16-token query block, KV head g), one wave per query
 * head of the group (and, up to 4 query heads per KV head, per half of the
 * key blocks: the halves merge at the end).  Per block of 16 key positions
 * the K and V rows come from the fp16 cache into LDS, and each wave
 * computes the scores and the output with an online softmax per query
 * column in log2 units (the decode step's attention does the same per lane
 * group).  A query's own key and value are its fp32 k/v (the cache holds
 * them in fp16), as in the token-sequential step: in the key block holding
 * a query's position its score is recomputed from the fp32 k row, and its
 * value enters as the fp16 row through the MFMA plus p (v32 - v16).  Key
 * positions past a query's own are masked.
 *
 * The products run on fp16 MFMA (v_mfma_f32_16x16x16_f16, fp32
 * accumulation): the cache rows are fp16 already, and each fp32
 * operand goes in as two fp16 parts, x = hi + lo (hi = fp16(x), lo =
 * fp16(x - hi)), so q.k = hi.k + lo.k and p.v = hi.v + lo.v keep ~22 bits of
 * every fp32 operand (each fp16 x fp16 product is exact in fp32).  p <= 1 is
 * scaled by 2^15 before the split, so p down to 2^-29 stays a normal fp16,
 * and the sums are unscaled at the end.  K is staged in LDS as it is
 * stored ([key][dim], rows padded 16 B against bank conflicts), V transposed
 * ([dim][key]): an MFMA lane takes 4 consecutive keys of one dim.
 *   S^T[key][q] = sum_d K[key][d] Q[q][d]   A = K, B = Q^T (16 dims a step)
 *   O^T[d][q]  += sum_key V^T[d][key] P^T[key][q]   A = V^T, B = P^T
 * P^T is the D layout of S^T (lane (g, q) holds keys 4g..4g+3), so it feeds
 * the second product without a transpose.  Only fp32 rounding differs from
 * the token-sequential step (sum orders, ~2^-22 per operand). */
template <int HD, int NREP, int SPLIT>
__global__ __launch_bounds__(64 * NREP * SPLIT) void k_pf_attn_h(const float* __restrict__ qkv, int qstride, int n_embed,
                                                         int kv_dim, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc, int pos0, int T,
                                                         float* __restrict__ att)
{
    static_assert(HD % 16 == 0 && HD <= 256, "16-dim output tiles");
    constexpr int NT = 64 * NREP * SPLIT, NTL = HD / 16, KST = HD + 8, VTS = 20, OST = HD + 4;
    constexpr float PS = 32768.0f;
    __shared__ __attribute__((aligned(16))) _Float16 s_kh[SPLIT][16 * KST];   /* K[key][d] */
    __shared__ __attribute__((aligned(16))) _Float16 s_vt[SPLIT][HD * VTS];   /* V^T[d][key] */
    __shared__ __attribute__((aligned(16))) float s_k32[16 * OST];    /* fp32 k / v of the block's 16 tokens */
    __shared__ __attribute__((aligned(16))) float s_v32[16 * OST];
    const int qb = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, r = (tid >> 6) % NREP, half = (tid >> 6) / NREP;
    const _Float16* __restrict__ s_k = s_kh[half];
    const _Float16* __restrict__ s_v = s_vt[half];
    const int col = lane & 15, grp = lane >> 4;
    const int t0 = qb * 16, tq = t0 + col, tqc = min(tq, T - 1);
    const int qpos = pos0 + tq;
    const int last = pos0 + min(t0 + 15, T - 1);   /* last key position this block reads */
    const float scale2 = 1.44269504088896341f / sqrtf((float)HD);

    /* B operand of S^T: Q[tq][16j + 4 grp + i], fp32 and as hi + lo */
    float qf[NTL][4];
    v4h qh[NTL], ql[NTL];
    const float* qrow = qkv + (size_t)tqc * qstride + (size_t)(g * NREP + r) * HD;
#pragma unroll
    for (int j = 0; j < NTL; j++) {
        const float4 v = *(const float4*)(qrow + 16 * j + 4 * grp);
        qf[j][0] = v.x; qf[j][1] = v.y; qf[j][2] = v.z; qf[j][3] = v.w;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16 h = (_Float16)qf[j][i];
            qh[j][i] = h;
            ql[j][i] = (_Float16)(qf[j][i] - (float)h);
        }
    }
    for (int i = tid; i < 16 * HD; i += NT) {
        const int tt = i / HD, d = i % HD;
        const float* row = qkv + (size_t)min(t0 + tt, T - 1) * qstride;
        s_k32[tt * OST + d] = row[n_embed + g * HD + d];
        s_v32[tt * OST + d] = row[n_embed + kv_dim + g * HD + d];
    }

    v4f o[NTL];
#pragma unroll
    for (int t = 0; t < NTL; t++) o[t] = (v4f){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;   /* l: this lane group's keys only, summed at the end */
    const int nkb = last / 16 + 1, nit = (nkb + SPLIT - 1) / SPLIT;
    constexpr int NPC = SPLIT * 16 * (HD / 8), NSTG = (NPC + NT - 1) / NT;
    /* the K/V pieces of the next step (piece i: 8 dims of one key of one
     * half's block), loaded while this step computes */
    struct Pieces {
        uint4 k[NSTG], v[NSTG];
    };
    auto stage_load = [&](int it) {
        Pieces P;
#pragma unroll
        for (int u = 0; u < NSTG; u++) {
            const int i = min(tid + u * NT, NPC - 1);
            const int hb = i / (16 * (HD / 8)), kk = (i / (HD / 8)) % 16, d8 = (i % (HD / 8)) * 8;
            const size_t off = (size_t)min((it * SPLIT + hb) * 16 + kk, last) * kv_dim + (size_t)g * HD + d8;
            P.k[u] = *(const uint4*)(kc + off);
            P.v[u] = *(const uint4*)(vc + off);
        }
        return P;
    };
    Pieces pc = stage_load(0);
    for (int it = 0; it < nit; it++) {
        __syncthreads();   /* the previous step's tiles are consumed */
#pragma unroll
        for (int u = 0; u < NSTG; u++) {
            const int i = tid + u * NT;
            if (NSTG * NT == NPC || i < NPC) {   /* (every thread has a piece when the pieces divide evenly) */
                const int hb = i / (16 * (HD / 8)), kk = (i / (HD / 8)) % 16, d8 = (i % (HD / 8)) * 8;
                *(uint4*)&s_kh[hb][kk * KST + d8] = pc.k[u];
                const uint4 vv = pc.v[u];
                uint16_t* vt = (uint16_t*)s_vt[hb] + d8 * VTS + kk;
                vt[0] = (uint16_t)(vv.x & 0xffffu);
                vt[VTS] = (uint16_t)(vv.x >> 16);
                vt[2 * VTS] = (uint16_t)(vv.y & 0xffffu);
                vt[3 * VTS] = (uint16_t)(vv.y >> 16);
                vt[4 * VTS] = (uint16_t)(vv.z & 0xffffu);
                vt[5 * VTS] = (uint16_t)(vv.z >> 16);
                vt[6 * VTS] = (uint16_t)(vv.w & 0xffffu);
                vt[7 * VTS] = (uint16_t)(vv.w >> 16);
            }
        }
        __syncthreads();
        pc = stage_load(min(it + 1, nit - 1));
        const int kb = it * SPLIT + half;
        if (kb >= nkb) continue;   /* the other half's last block (wave-uniform) */

        v4f sa = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NTL; j++) {
            const v4h a = *(const v4h*)(s_k + col * KST + 16 * j + 4 * grp);
            sa = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qh[j], sa, 0, 0, 0);
            sa = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ql[j], sa, 0, 0, 0);
        }
        float sv[4] = {sa[0], sa[1], sa[2], sa[3]};
        /* the block holds some query's own position: exact fp32 scores */
        const bool diag = kb * 16 + 15 >= pos0 + t0 && kb * 16 <= pos0 + t0 + 15;
        const int own = qpos - kb * 16;   /* 0..15 when this lane's query owns a key here */
        if (diag) {
            float e = 0.0f;
#pragma unroll
            for (int j = 0; j < NTL; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) e = __builtin_fmaf(qf[j][i], s_k32[col * OST + 16 * j + 4 * grp + i], e);
            e += lg_partner<4>(e);
            e += lg_partner<5>(e);
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (own == 4 * grp + i) sv[i] = e;
        }
        float bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sv[i] = kb * 16 + 4 * grp + i > qpos ? -INFINITY : sv[i] * scale2;
            bm = fmaxf(bm, sv[i]);
        }
        bm = fmaxf(bm, lg_partner<4>(bm));
        bm = fmaxf(bm, lg_partner<5>(bm));
        const float mn = fmaxf(m, bm);   /* finite: key 0 is in every query's range */
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        float pw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pw[i] = __builtin_amdgcn_exp2f(sv[i] - mn);
        l = __builtin_fmaf(l, alpha, (pw[0] + pw[1]) + (pw[2] + pw[3]));
        m = mn;
        float pown = 0.0f;   /* p of the own key, broadcast to the column's four lane groups */
        if (diag) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (own == 4 * grp + i) pown = pw[i];
            pown += lg_partner<4>(pown);
            pown += lg_partner<5>(pown);
        }
        /* P^T operand: the lane's keys 4 grp..+3, scaled, as hi + lo */
        v4h ph, pl;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float ps = pw[i] * PS;
            const _Float16 h = (_Float16)ps;
            ph[i] = h;
            pl[i] = (_Float16)(ps - (float)h);
        }
#pragma unroll
        for (int t = 0; t < NTL; t++) {
            o[t] *= alpha;
            const v4h a = *(const v4h*)(s_v + (16 * t + col) * VTS + 4 * grp);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pl, o[t], 0, 0, 0);
        }
        if (diag && own >= 0 && own < 16) {
            const float pso = pown * PS;
#pragma unroll
            for (int t = 0; t < NTL; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int d = 16 * t + 4 * grp + i;
                    o[t][i] = __builtin_fmaf(pso, s_v32[col * OST + d] - (float)s_v[d * VTS + own], o[t][i]);
                }
        }
    }
    if constexpr (SPLIT == 2) {
        /* the second half's (m, l, o) into the first half's lanes */
        __shared__ float s_x[NREP][2 + 4 * NTL][64];
        if (half == 1) {
            s_x[r][0][lane] = m;
            s_x[r][1][lane] = l;
#pragma unroll
            for (int t = 0; t < NTL; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) s_x[r][2 + 4 * t + i][lane] = o[t][i];
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = s_x[r][0][lane], mx = fmaxf(m, m1);
        const float a0 = __builtin_amdgcn_exp2f(m - mx), a1 = __builtin_amdgcn_exp2f(m1 - mx);
        l = lg_fma2(l, a0, s_x[r][1][lane], a1);
#pragma unroll
        for (int t = 0; t < NTL; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[t][i] = lg_fma2(o[t][i], a0, s_x[r][2 + 4 * t + i][lane], a1);
    }
    l += lg_partner<4>(l);
    l += lg_partner<5>(l);
    if (tq < T) {
        const float inv = 1.0f / (l * PS);
        float* out = att + (size_t)tq * n_embed + (size_t)(g * NREP + r) * HD;
#pragma unroll
        for (int t = 0; t < NTL; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) out[16 * t + 4 * grp + i] = o[t][i] * inv;
    }
}

int lg_prefill_attn_supported(int head_dim, int nrep)
{
    return (head_dim == 48 || head_dim == 64 || head_dim == 128) && nrep >= 1 && nrep <= 8;
}

static int launch_attn(const PfModel& M, const float* qkv, int qs, const uint16_t* kc, const uint16_t* vc, int T,
                       int pos0, float* att, hipStream_t s)
{
    const int nrep = M.n_heads / M.n_kv;
    if (!lg_prefill_attn_supported(M.head_dim, nrep)) {
        lg_set_error("prefill attention: head_dim %d with %d query heads per KV head", M.head_dim, nrep);
        return LG_ERR_TYPE;
    }
    const dim3 grid((T + 15) / 16, M.n_kv);
    /* two halves of the key blocks per query head up to 4 query heads per
     * KV head (8 waves); one at 8 (8 waves already) */
#define PFA(HD, NR)                                                                                          \
    hipLaunchKernelGGL((k_pf_attn_h<HD, NR, (NR <= 4 ? 2 : 1)>), grid, dim3(64 * NR * (NR <= 4 ? 2 : 1)), 0, s, \
                       qkv, qs, M.n_embed, M.kv_dim, kc, vc, pos0, T, att)
#define PFA_HD(HD)                    \
    switch (nrep) {                   \
    case 1: PFA(HD, 1); break;        \
    case 2: PFA(HD, 2); break;        \
    case 3: PFA(HD, 3); break;        \
    case 4: PFA(HD, 4); break;        \
    case 5: PFA(HD, 5); break;        \
    case 6: PFA(HD, 6); break;        \
    case 7: PFA(HD, 7); break;        \
    default: PFA(HD, 8); break;       \
    }
    switch (M.head_dim) {
    case 48: PFA_HD(48); break;
    case 64: PFA_HD(64); break;
    default: PFA_HD(128); break;
    }
#undef PFA_HD
#undef PFA
    return lg_check_launch("prefill attention");
}

/* one pass's quantized activation of every token into the trace, as the
 * reference's blocks (block_q8_K: d, qs[256], bsums[16]; block_q8_0: fp16 d,
 * qs[32]): block b of token t */
template <int QT>
__global__ __launch_bounds__(64) void k_pf_trace(PfQ8K q, int n, uint8_t* __restrict__ tr, size_t tok_stride)
{
    const int b = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    constexpr int QK = QT == LG_Q8_K ? 256 : 32, BS = QT == LG_Q8_K ? LG_BS_Q8_K : LG_BS_Q8_0;
    uint8_t* o = tr + (size_t)t * tok_stride + (size_t)b * BS;
    const int8_t* qs = q.qs + (size_t)t * n + (size_t)b * QK;
    const int off = QT == LG_Q8_K ? 4 : 2;
    for (int i = lane; i < QK; i += 64) o[off + i] = (uint8_t)qs[i];
    if (QT == LG_Q8_K) {
        if (lane < 16) {
            const int16_t v = q.bs[((size_t)t * (n >> 8) + b) * 16 + lane];
            __builtin_memcpy(o + 260 + 2 * lane, &v, 2);
        }
        if (lane == 0) {
            const float d = q.d[(size_t)b * q.tld + t];
            __builtin_memcpy(o, &d, 4);
        }
    } else if (lane == 0) {
        const uint16_t dh = lg_f2h(q.d[(size_t)b * q.tld + t]);
        __builtin_memcpy(o, &dh, 2);
    }
}

int lg_prefill_layers(const PfModel& M, PfBuffers& B, int T, int pos0, hipStream_t s)
{
    if (T <= 0 || T > B.tmax || pos0 < 0 || pos0 + T > M.n_ctx) {
        lg_set_error("prefill: %d tokens at %d (buffers for %d, context %d)", T, pos0, B.tmax, M.n_ctx);
        return LG_ERR_STATE;
    }
    const int ne = M.n_embed, kvd = M.kv_dim, qs = ne + 2 * kvd, nff = M.n_ff;
    const size_t tstride = (size_t)(4 * M.n_layers + 1) * B.trace_stride;
    /* activation forms the matrices take: bit 0 Q8_K, bit 1 Q8_0, bit 2 F32 */
    auto fam = [](const PfMat& W) {
        const int at = lg_prefill_act_type(W.type);
        return at == LG_Q8_K ? 1 : at == LG_Q8_0 ? 2 : 4;
    };
    auto trace = [&](int f, int n, int k) -> int {
        if (!B.trace || !(f & 3)) return LG_OK;   /* fp32 activations are not quantized: nothing to record */
        uint8_t* tr = B.trace + (size_t)k * B.trace_stride;
        if (f & 1) hipLaunchKernelGGL(k_pf_trace<LG_Q8_K>, dim3(n / 256, T), dim3(64), 0, s, B.qk, n, tr, tstride);
        else hipLaunchKernelGGL(k_pf_trace<LG_Q8_0>, dim3(n / 32, T), dim3(64), 0, s, B.q0, n, tr, tstride);
        return lg_check_launch("prefill trace");
    };
    /* rmsnorm (w) and quantization of T rows of x in each form f asks for;
     * the trace records the Q8_K form when both are made, as a step does */
    auto quant = [&](int f, const float* x, const float* w, int n, int k) -> int {
        int rc;
        if ((f & 1) && (rc = lg_prefill_quantize(LG_Q8_K, x, n, w, M.eps, n, T, B.qk, s))) return rc;
        if ((f & 2) && (rc = lg_prefill_quantize(LG_Q8_0, x, n, w, M.eps, n, T, B.q0, s))) return rc;
        if ((f & 4) && (rc = lg_prefill_quantize(LG_F32, x, n, w, M.eps, n, T, B.qf, s))) return rc;
        return trace(f, n, k);
    };
    auto gemm = [&](const PfMat& W, int cols, float* o, int ldo, int acc) {
        const int f = fam(W);
        return lg_prefill_gemm(W.type, W.w, W.rsz, W.rows, cols, f == 1 ? B.qk : f == 2 ? B.q0 : B.qf, T, o, ldo, acc, s);
    };
    int rc;
    hipLaunchKernelGGL(k_pf_embed, dim3(T), dim3(256), 0, s, M.embd_t, M.embd, M.embd_rsz, B.toks, ne, B.x);
    if ((rc = lg_check_launch("prefill embedding"))) return rc;
    for (int l = 0; l < M.n_layers; l++) {
        const PfLayer& L = M.layers[l];
        uint16_t* kc = M.kc + (size_t)l * M.n_ctx * kvd;
        uint16_t* vc = M.vc + (size_t)l * M.n_ctx * kvd;
        /* attention branch */
        const int f_qkv = L.qkv_fused ? fam(L.qkv) : fam(L.q) | fam(L.k) | fam(L.v);
        if ((rc = quant(f_qkv, B.x, L.att_norm, ne, 4 * l))) return rc;
        if (L.qkv_fused) {
            if ((rc = gemm(L.qkv, ne, B.qkv, qs, 0))) return rc;
        } else {
            if ((rc = gemm(L.q, ne, B.qkv, qs, 0))) return rc;
            if ((rc = gemm(L.k, ne, B.qkv + ne, qs, 0))) return rc;
            if ((rc = gemm(L.v, ne, B.qkv + ne + kvd, qs, 0))) return rc;
        }
        const int waves = M.n_heads + M.n_kv;
        hipLaunchKernelGGL(k_pf_qk_rope_kv, dim3((waves + 3) / 4, T), dim3(256), 0, s, B.qkv, qs, ne, kvd, L.q_norm,
                           L.k_norm, M.n_heads, M.n_kv, M.head_dim, M.rope_dim, pos0, M.rope_freq, M.eps, kc, vc);
        if ((rc = lg_check_launch("prefill qk-norm/rope/kv"))) return rc;
        if ((rc = launch_attn(M, B.qkv, qs, kc, vc, T, pos0, B.att, s))) return rc;
        if ((rc = quant(fam(L.ao), B.att, nullptr, ne, 4 * l + 1))) return rc;
        if ((rc = gemm(L.ao, ne, B.x, ne, 1))) return rc;
        /* FFN branch */
        const int f_ug = L.ug_fused ? fam(L.ug) : fam(L.up) | fam(L.gate);
        if ((rc = quant(f_ug, B.x, L.ffn_norm, ne, 4 * l + 2))) return rc;
        if (L.ug_fused) {
            if ((rc = gemm(L.ug, ne, B.ug, 2 * nff, 0))) return rc;
        } else {
            if ((rc = gemm(L.up, ne, B.ug, 2 * nff, 0))) return rc;
            if ((rc = gemm(L.gate, ne, B.ug + nff, 2 * nff, 0))) return rc;
        }
        const int f_d = fam(L.down);
        const dim3 sg((nff + 255) / 256, T);
        if (f_d == 1) hipLaunchKernelGGL(k_pf_swiglu_quant<LG_Q8_K>, sg, dim3(64), 0, s, B.ug, nff, B.qk);
        else if (f_d == 2) hipLaunchKernelGGL(k_pf_swiglu_quant<LG_Q8_0>, sg, dim3(64), 0, s, B.ug, nff, B.q0);
        else hipLaunchKernelGGL(k_pf_swiglu_quant<LG_F32>, sg, dim3(64), 0, s, B.ug, nff, B.qf);
        if ((rc = lg_check_launch("prefill swiglu"))) return rc;
        if ((rc = trace(f_d, nff, 4 * l + 3))) return rc;
        if ((rc = gemm(L.down, nff, B.x, ne, 1))) return rc;
    }
    return LG_OK;
}
