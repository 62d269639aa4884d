/* lg_attn.hip -- GQA decode attention over the fp16 KV cache for gfx950
 * (the inline attention block of inference(), fast/ligguf_fast_qk.cpp:64-105,
 * with softmax of fast/lil_math.cpp:964-976).
 *
 * Split over the sequence ("flash-decoding"): workgroup (chunk c, KV head
 * kh) takes positions [c*CH, min((c+1)*CH, pos+1)) and all NREP query heads
 * that share kh, so every K/V row is read from HBM once.  The partials
 * (m in log2 units, l, o) of each chunk go to the workspace; k_attn_merge
 * rescales them by 2^(m_c - M) and divides by the total, which equals the
 * reference's single-pass softmax.  t == pos takes the fp32 k and v of this
 * step (fast/ligguf_fast_qk.cpp:77-79, 98-99): the cache row is not written
 * yet.
 *
 * k_attn_tile (head_dim 64, 128, 256): one pass, 4 waves.  Each wave streams
 * its own rows of every tile of TP positions (TP/4 per wave) into LDS with
 * direct-to-LDS loads (global_load_lds_dwordx4), NBUF tiles deep, counting
 * its waits by hand; the rows never pass through registers, and since no
 * wave reads another's rows the loop has no workgroup barrier.  Per tile a
 * wave takes the scores by LPP = HD/8 lanes per position (8 dims each, the
 * 16-lane tree of the three-pass kernel), the online softmax in log2 units
 * one (head, position) per lane (v_exp_f32; one rescale of the running sums
 * per head and tile), then p.V by the position lanes.  The waves merge at
 * the end.
 *
 * k_attn_unit (head_dim 64, 128, 256, up to 4096 positions): one query
 * head per workgroup, K/V rows through registers, merged per head by
 * k_attn_unit_merge -- NREP times the workgroups of k_attn_tile, which
 * wins at longer contexts by reading each row once per KV head.
 *
 * k_attn_split (head_dim 48, and position 0): three passes per chunk.
 * A K/V row of one head is HD fp16 = 2*HD bytes; LPP lanes split it (DPL
 * dims each), so a wave covers 64/LPP positions per step.
 *   pass 1: scores s[h][t] = q_h . k_t * scale into LDS;
 *   pass 2: chunk max m and p = exp(s - m), l = sum p;
 *   pass 3: o[h] = sum_t p[h][t] v_t.
 */
#include <math.h>

#include <mutex>

#include "lg_common.h"

#define LG_ATTN_MAX_CHUNK 1024

/* chunk length for a context of ctx positions: about 128 chunks (with 8 KV
 * heads, 1024 workgroups: four per CU), between 64 and LG_ATTN_MAX_CHUNK
 * positions, multiple of 64 */
static int attn_chunk(int ctx)
{
    int c = (ctx + 127) / 128;
    c = (c + 63) / 64 * 64;
    if (c < 64) c = 64;
    if (c > LG_ATTN_MAX_CHUNK) c = LG_ATTN_MAX_CHUNK;
    return c;
}

/* k_attn_tile: 4 waves; per tile each lane holds two 16-byte pieces of K
 * (and of V), fewer when the softmax would need more than one lane per
 * (query head, position): TPW positions per wave, TP = 4 TPW per tile.
 * Chunks of a whole number of tiles, 64 of them (fewer for short contexts:
 * at least 64 positions each), more past 4096 positions per chunk */
#define LG_ATTN_TW 4
#define LG_ATTN_TCH 64
#define LG_ATTN_TMAX 4096
__host__ __device__ constexpr int attn_tpw(int hd, int nrep)
{
    /* a whole number of position steps (512 / hd positions per wave step) */
    return ((2 * 64 * 8 / hd) < (64 / nrep) ? (2 * 64 * 8 / hd) : (64 / nrep)) / (512 / hd) * (512 / hd);
}
__host__ __device__ constexpr int attn_tp(int hd, int nrep) { return LG_ATTN_TW * attn_tpw(hd, nrep); }

static bool attn_tiled(int head_dim, int pos)
{
    return pos > 0 && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

static void attn_tile_split(int ctx, int hd, int nrep, int* chunk, int* nch)
{
    const int tp = attn_tp(hd, nrep);
    int n = (ctx + 63) / 64;
    if (n > LG_ATTN_TCH) n = LG_ATTN_TCH;
    const int nmin = (ctx + LG_ATTN_TMAX - 1) / LG_ATTN_TMAX;
    if (n < nmin) n = nmin;
    int c = (ctx + n - 1) / n;
    c = (c + tp - 1) / tp * tp;
    *chunk = c;
    *nch = (ctx + c - 1) / c;
}

/* chunks of a context: never fewer for a longer context, so a workspace
 * sized for the last position serves every earlier one */
static int attn_nch_bound(int head_dim, int pos)
{
    const int ctx = pos + 1;
    if (attn_tiled(head_dim, pos)) {
        const int nmin = (ctx + LG_ATTN_TMAX - 1) / LG_ATTN_TMAX;
        return nmin > LG_ATTN_TCH ? nmin : LG_ATTN_TCH;
    }
    /* attn_chunk: chunks of 64 keys up to 8192 keys (at most 128 chunks),
     * at most 128 chunks up to 131072 keys, chunks of LG_ATTN_MAX_CHUNK past */
    const int small = (ctx + 63) / 64 < 128 ? (ctx + 63) / 64 : 128;
    const int over = (ctx + LG_ATTN_MAX_CHUNK - 1) / LG_ATTN_MAX_CHUNK;
    return over > small ? over : small;
}

size_t lg_attn_ws_bytes(int n_heads, int head_dim, int pos)
{
    if (n_heads <= 0 || head_dim <= 0 || pos < 0) return 0;
    /* a workspace sized for pos serves every earlier position (for the
     * tiled head sizes that includes position 0, one chunk of the
     * three-pass kernel) */
    const int nb = attn_nch_bound(head_dim, pos);
    return (size_t)n_heads * nb * (head_dim + 2) * sizeof(float);
}

template <int DPL>
__device__ __forceinline__ void load_half_row(const uint16_t* __restrict__ p, float out[DPL])
{
    if constexpr (DPL == 8) {
        const uint4 v = lg_ld<uint4>((const uint8_t*)p);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[2 * i] = lg_h2f((uint16_t)(u[i] & 0xffffu));
            out[2 * i + 1] = lg_h2f((uint16_t)(u[i] >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < DPL; i++) out[i] = lg_h2f(p[i]);
    }
}

template <int DPL>
__device__ __forceinline__ void load_f32_row(const float* __restrict__ p, float out[DPL])
{
#pragma unroll
    for (int i = 0; i < DPL; i++) out[i] = p[i];
}

/* workspace layout per (kv head kh, chunk c): NREP m (log2 units), NREP l,
 * NREP*HD o; i.e. per query head h = kh*NREP + r: index ((kh*nch + c)*NREP + r) */
template <int HD, int NREP, int LPP>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ q, const float* __restrict__ kcur,
                                                    const float* __restrict__ vcur, const uint16_t* __restrict__ kc,
                                                    const uint16_t* __restrict__ vc, int kv_dim, int pos, int chunk,
                                                    int nch, float scale, float* __restrict__ ws)
{
    constexpr int DPL = HD / LPP;
    constexpr int PPW = 64 / LPP;      /* positions per wave step */
    constexpr int PPB = 4 * PPW;       /* positions per workgroup step */
    __shared__ float s_sc[NREP * LG_ATTN_MAX_CHUNK];
    __shared__ float s_red[4 * NREP * HD];
    __shared__ float s_m[4 * NREP];

    const int c = blockIdx.x, kh = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane & (LPP - 1), grp = lane / LPP;
    const int t0 = c * chunk;
    int t1 = t0 + chunk;
    if (t1 > pos + 1) t1 = pos + 1;
    const int nt = t1 - t0;

    float qr[NREP][DPL];
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) qr[r][i] = q[(size_t)(kh * NREP + r) * HD + gl * DPL + i];

    /* pass 1: scores, U steps of rows loaded before any is used (positions
     * past the chunk load its first row and are not stored) */
    constexpr int U = 4;
    for (int tb = 0; tb < nt; tb += U * PPB) {
        float kv[U][DPL];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            const int t = tl < nt ? t0 + tl : t0;
            if (t == pos) load_f32_row<DPL>(kcur + kh * HD + gl * DPL, kv[u]);
            else load_half_row<DPL>(kc + (size_t)t * kv_dim + kh * HD + gl * DPL, kv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
#pragma unroll
            for (int r = 0; r < NREP; r++) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < DPL; i++) s += qr[r][i] * kv[u][i];
                s = lg_group_sum<LPP>(s);
                if (gl == 0 && tl < nt) s_sc[r * LG_ATTN_MAX_CHUNK + tl] = s * scale;
            }
        }
    }
    __syncthreads();

    /* pass 2: chunk max and exponentials (each wave scans for all heads) */
    float m[NREP], l[NREP];
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        float mx = -INFINITY;
        for (int i = threadIdx.x; i < nt; i += 256) mx = fmaxf(mx, s_sc[r * LG_ATTN_MAX_CHUNK + i]);
        mx = lg_group_max<64>(mx);
        if (lane == 0) s_m[wave * NREP + r] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        m[r] = fmaxf(fmaxf(s_m[r], s_m[NREP + r]), fmaxf(s_m[2 * NREP + r], s_m[3 * NREP + r]));
        float sum = 0.0f;
        for (int i = threadIdx.x; i < nt; i += 256) {
            const float p = expf(s_sc[r * LG_ATTN_MAX_CHUNK + i] - m[r]);
            s_sc[r * LG_ATTN_MAX_CHUNK + i] = p;
            sum += p;
        }
        l[r] = sum;   /* partial; reduced below */
    }
    __syncthreads();

    /* pass 3: p . V */
    float o[NREP][DPL];
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) o[r][i] = 0.0f;
    for (int tb = 0; tb < nt; tb += U * PPB) {
        float vv[U][DPL];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            const int t = tl < nt ? t0 + tl : t0;
            if (t == pos) load_f32_row<DPL>(vcur + kh * HD + gl * DPL, vv[u]);
            else load_half_row<DPL>(vc + (size_t)t * kv_dim + kh * HD + gl * DPL, vv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tl = tb + u * PPB + wave * PPW + grp;
            if (tl < nt) {
#pragma unroll
                for (int r = 0; r < NREP; r++) {
                    const float p = s_sc[r * LG_ATTN_MAX_CHUNK + tl];
#pragma unroll
                    for (int i = 0; i < DPL; i++) o[r][i] += p * vv[u][i];
                }
            }
        }
    }
    /* reduce o over the position groups of the wave, then over waves */
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) {
            float v = o[r][i];
#pragma unroll
            for (int off = LPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
            o[r][i] = v;
        }
    if (grp == 0) {
#pragma unroll
        for (int r = 0; r < NREP; r++)
#pragma unroll
            for (int i = 0; i < DPL; i++) s_red[(wave * NREP + r) * HD + gl * DPL + i] = o[r][i];
    }
    /* l: block sum per head */
#pragma unroll
    for (int r = 0; r < NREP; r++) {
        float v = lg_group_sum<64>(l[r]);
        l[r] = v;
    }
    __syncthreads();
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NREP; r++) s_m[wave * NREP + r] = l[r];
    }
    __syncthreads();
    float* out = ws + ((size_t)kh * nch + c) * NREP * (HD + 2);
    for (int i = threadIdx.x; i < NREP * HD; i += 256) {
        const int r = i / HD, dd = i % HD;
        out[2 * NREP + r * HD + dd] = s_red[(0 * NREP + r) * HD + dd] + s_red[(1 * NREP + r) * HD + dd] +
                                      s_red[(2 * NREP + r) * HD + dd] + s_red[(3 * NREP + r) * HD + dd];
    }
    if (threadIdx.x < NREP) {
        const int r = threadIdx.x;
        out[r] = m[r] * 1.44269504088896341f;   /* log2 units, as k_attn_tile's */
        out[NREP + r] = s_m[r] + s_m[NREP + r] + s_m[2 * NREP + r] + s_m[3 * NREP + r];
    }
}

/* 16 bytes from global memory to LDS at m0 + 16 * lane (m0 wave-uniform);
 * completion counts in vmcnt like any vector load, and nothing but an
 * explicit s_waitcnt waits for it.  m0 is named as clobbered although the
 * compiler reserves it (it warns): none of these kernels uses m0 otherwise
 * (checked in their ISA). */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void attn_dma16(const void* g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void attn_wait_vm()
{
    static_assert(N >= 0 && N <= 63, "vmcnt field");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* barrier: this wave's LDS operations done, then every wave */
__device__ __forceinline__ void attn_bar()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* the 8 halves of a 16-byte piece, each converted inside the fma that uses
 * it (v_fma_mix_f32: the conversion is exact, the fma the same) */
struct AttnH8 {
    _Float16 h[8];
    __device__ __forceinline__ void set(uint4 u) { __builtin_memcpy(h, &u, 16); }
    __device__ __forceinline__ float f(int i) const { return (float)h[i]; }
};

/* workspace layout as k_attn_split's; LG_ATTN_TW waves, chunk a multiple of TP */
template <int HD, int NREP>
__global__ __launch_bounds__(LG_ATTN_TW * 64) void k_attn_tile(const float* __restrict__ q, const float* __restrict__ kcur,
                                                   const float* __restrict__ vcur, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, int kv_dim, int pos, int chunk,
                                                   int nch, float scale2, float* __restrict__ ws)
{
    constexpr int NW = LG_ATTN_TW;
    constexpr int TPW = attn_tpw(HD, NREP);  /* positions per wave and tile */
    constexpr int TP = NW * TPW;             /* positions per tile */
    constexpr int CPR = HD * 2 / 16;         /* 16-byte pieces per fp16 row */
    constexpr int PW = TPW * CPR;            /* pieces per wave, tile and matrix */
    constexpr int NBUF = 4;
    constexpr int IPW = PW / 64;             /* DMA instructions per wave, tile and matrix */
    constexpr int IPT = 2 * IPW;
    constexpr int LPP = HD / 8;              /* lanes per position in the scores and p.V */
    constexpr int PPW = 64 / LPP;            /* positions per wave step */
    constexpr int SPT = TPW / PPW;           /* steps per wave and tile */
    constexpr int HP = (NREP * HD + 2 * HD) * 4 / 16;   /* pieces of q, k, v of this step */
    constexpr int HI = (HP + NW * 64 - 1) / (NW * 64);   /* their instructions per wave */
    static_assert(PW % 64 == 0 && IPW >= 1, "tile in whole wave instructions");
    static_assert(TPW % PPW == 0 && NREP * TPW <= 64, "wave geometry");
    static_assert(HI + (NBUF - 2) * IPT <= 63, "vmcnt range");
    /* each wave's own rows of every buffered tile: no wave reads another's */
    __shared__ __attribute__((aligned(16))) uint4 s_kv[2][NBUF][NW][PW];   /* K, V */
    __shared__ __attribute__((aligned(16))) float s_head[HI * NW * 64 * 4];   /* q (NREP x HD), k, v */
    __shared__ float s_s[NW][NREP * TPW];   /* per wave: scores, then exponentials */
    __shared__ float s_a[NW][NREP];         /* per wave: rescale of the running sums */
    __shared__ float s_ml[NW][2 * NREP];
    static_assert(NW * NREP * HD * 4 <= (int)sizeof(s_kv), "the waves' outputs fit the tile buffers");

    const int c = blockIdx.x, kh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gl = lane & (LPP - 1), grp = lane / LPP;
    const int t0 = c * chunk;
    const int t1 = min(t0 + chunk, pos + 1);
    const int ntiles = (t1 - t0 + TP - 1) / TP;
    const uint32_t lds_k = (uint32_t)(uintptr_t)&s_kv[0][0][wave][0], lds_v = (uint32_t)(uintptr_t)&s_kv[1][0][wave][0];

    /* q of the group's heads, k and v of this step, shared by the waves
     * (pieces past the end load the last one again) */
#pragma unroll
    for (int k = 0; k < HI; k++) {
        const int pc = min((k * NW + wave) * 64 + lane, HP - 1);
        const int f = pc * 4;                  /* float index in s_head */
        const float* src = f < NREP * HD ? q + (size_t)kh * NREP * HD + f
                         : f < NREP * HD + HD ? kcur + (size_t)kh * HD + (f - NREP * HD)
                                              : vcur + (size_t)kh * HD + (f - NREP * HD - HD);
        attn_dma16(src, __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)s_head + (k * NW + wave) * 1024));
    }
    /* this wave's rows of tile j (positions t0 + j*TP + wave*TPW ..) into
     * buffer j % NBUF.  Rows past the chunk, past the context and row pos
     * (not in the cache yet) load the chunk's last cache row instead and are
     * not used. */
    const int tend = min(t1, pos);        /* the tiles' positions: [t0, tend) from the cache */
    const int tlast = tend - 1;           /* the last row read from the cache */
    auto issue = [&](int j) {
        const int b = j % NBUF;
#pragma unroll
        for (int k = 0; k < IPW; k++) {
            const int pc = k * 64 + lane;
            const int row = pc / CPR, col = pc % CPR;
            const int t = min(t0 + j * TP + wave * TPW + row, tlast);
            const size_t o = (size_t)t * kv_dim + (size_t)kh * HD + col * 8;
            const uint32_t off = (uint32_t)((b * NW * PW + k * 64) * 16);
            attn_dma16(kc + o, __builtin_amdgcn_readfirstlane(lds_k + off));
            attn_dma16(vc + o, __builtin_amdgcn_readfirstlane(lds_v + off));
        }
    };
#pragma unroll
    for (int j = 0; j < NBUF - 1; j++) issue(j);

    float qr[NREP][8];
    float o[NREP][8];
    float m_run = -INFINITY, l_run = 0.0f;   /* lanes i < NREP*TPW: head i / TPW (log2 units) */
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int i = 0; i < 8; i++) o[r][i] = 0.0f;
    const int sr = lane / TPW, sp = lane % TPW;   /* this lane's (head, position) in the softmax */
    const bool slane = lane < NREP * TPW;

    for (int i = 0; i < ntiles; i++) {
        attn_wait_vm<(NBUF - 2) * IPT>();   /* this wave's tile i (and its head pieces) */
        if (i == 0) {
            attn_bar();                      /* every wave's head pieces */
#pragma unroll
            for (int r = 0; r < NREP; r++)
#pragma unroll
                for (int d = 0; d < 8; d++) qr[r][d] = s_head[r * HD + gl * 8 + d];
        }
        /* the buffer of tile i - 1 (read by this wave only) takes tile
         * i + NBUF - 1 once this wave's reads of it are done */
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + NBUF - 1);
        const int b = i % NBUF;
        const int tb = t0 + i * TP + wave * TPW;   /* first position of this wave's share */
        /* scores (log2 units); position pos is taken after the tiles */
#pragma unroll
        for (int st = 0; st < SPT; st++) {
            const int pl = st * PPW + grp;          /* position in the wave's share */
            const int t = tb + pl;
            AttnH8 kh8;
            kh8.set(s_kv[0][b][wave][pl * CPR + gl]);
#pragma unroll
            for (int r = 0; r < NREP; r++) {
                float sc = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) sc = __builtin_fmaf(kh8.f(d), qr[r][d], sc);
                sc = lg_group_sum<LPP>(sc);
                if (gl == 0) s_s[wave][r * TPW + pl] = t < tend ? sc * scale2 : -INFINITY;
            }
        }
        __builtin_amdgcn_wave_barrier();
        /* softmax: lane (head sr, position sp); tile max and sum over the
         * TPW lanes of the head */
        if (slane) {
            const float sv = s_s[wave][sr * TPW + sp];
            const float mn = fmaxf(m_run, lg_group_max<TPW>(sv));
            const float a = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - mn);
            const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv - mn);
            l_run = l_run * a + lg_group_sum<TPW>(p);
            m_run = mn;
            s_s[wave][sr * TPW + sp] = p;
            if (sp == 0) s_a[wave][sr] = a;
        }
        __builtin_amdgcn_wave_barrier();
        /* p.V; the running sums rescale only when a head's maximum moved
         * (a is 1 otherwise: the branch is uniform over the wave) */
#pragma unroll
        for (int r = 0; r < NREP; r++) {
            const float ar = s_a[wave][r];
            if (ar != 1.0f) {
#pragma unroll
                for (int d = 0; d < 8; d++) o[r][d] *= ar;
            }
        }
#pragma unroll
        for (int st = 0; st < SPT; st++) {
            const int pl = st * PPW + grp;
            AttnH8 vh8;
            vh8.set(s_kv[1][b][wave][pl * CPR + gl]);
#pragma unroll
            for (int r = 0; r < NREP; r++) {
                const float p = s_s[wave][r * TPW + pl];
#pragma unroll
                for (int d = 0; d < 8; d++) o[r][d] = __builtin_fmaf(vh8.f(d), p, o[r][d]);
            }
        }
    }
    attn_wait_vm<0>();   /* the trailing tiles (not used) land before the buffers are reused */
    /* position pos (the chunk holding it, wave 0): this step's fp32 k and v,
     * one more online-softmax step on the wave's state; every position
     * group computes it, the groups' p.V terms are summed below, so only
     * group 0 adds its o term */
    if (wave == 0 && pos < t1) {
#pragma unroll
        for (int r = 0; r < NREP; r++) {
            float sc = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) sc = __builtin_fmaf(s_head[NREP * HD + gl * 8 + d], qr[r][d], sc);
            const float sv = lg_group_sum<LPP>(sc) * scale2;
            const float mr = __shfl(m_run, r * TPW, 64), lr = __shfl(l_run, r * TPW, 64);
            const float mn = fmaxf(mr, sv);
            const float a = mr == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mr - mn);
            const float p = __builtin_amdgcn_exp2f(sv - mn);
#pragma unroll
            for (int d = 0; d < 8; d++)
                o[r][d] = __builtin_fmaf(grp == 0 ? p : 0.0f, s_head[NREP * HD + HD + gl * 8 + d], o[r][d] * a);
            if (slane && sr == r) {
                m_run = mn;
                l_run = lr * a + p;
            }
        }
    }
    /* the wave's position groups share its running max: plain sums over
     * the lanes holding the same dims (lane ^ LPP, ^ 2 LPP, ..) */
#pragma unroll
    for (int r = 0; r < NREP; r++)
#pragma unroll
        for (int d = 0; d < 8; d++) {
            float v = o[r][d];
            if constexpr (LPP <= 8) v += __shfl_xor(v, 8, 64);
            if constexpr (LPP <= 16) v += lg_partner<4>(v);
            if constexpr (LPP <= 32) v += lg_partner<5>(v);
            o[r][d] = v;
        }
    attn_bar();
    float* s_o = (float*)&s_kv[0][0][0][0];   /* [NW waves][NREP][HD] */
    if (grp == 0) {
#pragma unroll
        for (int r = 0; r < NREP; r++)
#pragma unroll
            for (int d = 0; d < 8; d++) s_o[(wave * NREP + r) * HD + gl * 8 + d] = o[r][d];
    }
    if (slane && sp == 0) {
        s_ml[wave][sr] = m_run;
        s_ml[wave][NREP + sr] = l_run;
    }
    attn_bar();
    float* out = ws + ((size_t)kh * nch + c) * NREP * (HD + 2);
    for (int k = tid; k < NREP * HD; k += NW * 64) {
        const int r = k / HD, d = k % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, s_ml[w][r]);
        float O = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float mw = s_ml[w][r];
            const float wt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            O += s_o[(w * NREP + r) * HD + d] * wt;
            L += s_ml[w][NREP + r] * wt;
        }
        out[2 * NREP + r * HD + d] = O;
        if (d == 0) {
            out[r] = M;
            out[NREP + r] = L;
        }
    }
}

/* one workgroup of 256 per query head: merge the chunk partials.  The
 * chunk weights 2^(m_c - M) and the total L once (threads over chunks,
 * weights of the first LG_ATTN_MERGE_W chunks kept in LDS), then each thread
 * sums one dim over a share of the chunks (PARTS threads per dim, their
 * loads issued together) and the shares add in LDS. */
#define LG_ATTN_MERGE_W 1024
template <int HD, int NREP>
__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ ws, int nch, float* __restrict__ out)
{
    constexpr int PARTS = HD >= 256 ? 1 : 256 / HD;
    constexpr int U = 8;
    __shared__ float s_w[LG_ATTN_MERGE_W];
    __shared__ float s_red[8];
    __shared__ float s_acc[PARTS][HD];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int kh = h / NREP, r = h % NREP;
    const size_t stride = (size_t)NREP * (HD + 2);
    const float* base = ws + (size_t)kh * nch * stride;
    float M = -INFINITY;
    for (int c = tid; c < nch; c += 256) M = fmaxf(M, base[c * stride + r]);
    M = lg_group_max<64>(M);
    if ((tid & 63) == 0) s_red[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float L = 0.0f;
    for (int c = tid; c < nch; c += 256) {
        const float w = __builtin_amdgcn_exp2f(base[c * stride + r] - M);
        if (c < LG_ATTN_MERGE_W) s_w[c] = w;
        L += base[c * stride + NREP + r] * w;
    }
    L = lg_group_sum<64>(L);
    __syncthreads();
    if ((tid & 63) == 0) s_red[4 + (tid >> 6)] = L;
    __syncthreads();
    L = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
    for (int d0 = 0; d0 < HD; d0 += 256 / PARTS) {
        const int d = d0 + tid % (256 / PARTS), part = tid / (256 / PARTS);
        float acc = 0.0f;
        if (d < HD) {
            const float* col = base + 2 * NREP + r * HD + d;
            for (int c0 = part; c0 < nch; c0 += PARTS * U) {
                float v[U], w[U];
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int c = min(c0 + u * PARTS, nch - 1);
                    v[u] = col[c * stride];
                    w[u] = c < LG_ATTN_MERGE_W ? s_w[c] : __builtin_amdgcn_exp2f(base[c * stride + r] - M);
                }
#pragma unroll
                for (int u = 0; u < U; u++)
                    if (c0 + u * PARTS < nch) acc += v[u] * w[u];
            }
            s_acc[part][d] = acc;
        }
        __syncthreads();
        if (part == 0 && d < HD) {
            float t = s_acc[0][d];
#pragma unroll
            for (int k = 1; k < PARTS; k++) t += s_acc[k][d];
            out[(size_t)h * HD + d] = t / L;
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------------ */
/* k_attn_unit (head_dim 64, 128, 256): one query head per workgroup.   */
/* ------------------------------------------------------------------ */
/* Contexts up to LG_ATTN_UNIT_CTX positions.  Unit (query head h, chunk c)
 * takes positions [c*chunk, min((c+1)*chunk, pos+1)) in one pass: 4 waves,
 * LPP = HD/8 lanes per position (8 dims each), PPB positions per workgroup
 * step, the K and V pieces of H steps per register batch, two batches in
 * flight; per position an online-softmax step of the lane group (log2
 * units).  Lane groups merge by lane permutes, waves in LDS, and the unit's
 * partial (m, l, o) goes to the workspace; k_attn_unit_merge merges each
 * head's chunks.  NREP times as many workgroups as k_attn_tile's (at least
 * 256 at 32 query heads); the NREP units of a (KV head, chunk) read the same
 * rows, and their workgroup indices differ by multiples of 8, so they run
 * together on one XCD and share its L2.  Past LG_ATTN_UNIT_CTX positions
 * k_attn_tile, which reads each row once per KV head, is faster (measured:
 * 8.3 / 14.6 / 61 us at 512 / 4096 / 32768 positions and 32 / 8 heads of
 * 128, against 9.6 / 15.3 / 38.5 for k_attn_tile + k_attn_merge). */
#define LG_ATTN_UNIT_MAX_NCH 16
#define LG_ATTN_UNIT_CTX 4096
#define LG_ATTN_UNIT_H 8   /* steps per register batch */

__device__ __forceinline__ float attn_dpp_ror8(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));   /* row_ror:8 */
}

/* combine two online-softmax states (m in log2 units; m = -inf: empty) */
__device__ __forceinline__ void attn_osm_merge(float& m, float& l, float* o, float m2, float l2, const float* o2)
{
    const float mn = fmaxf(m, m2);
    const float a = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
    const float b = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - mn);
    l = lg_fma2(l, a, l2, b);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = lg_fma2(o[i], a, o2[i], b);
    m = mn;
}

template <int HD, int NREP>
__global__ __launch_bounds__(256) void k_attn_unit(const float* __restrict__ q, const float* __restrict__ kcur,
                                                   const float* __restrict__ vcur, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, int n_kv, int pos, int chunk,
                                                   int nch, float scale2, float* __restrict__ ws)
{
    constexpr int NW = 4, LPP = HD / 8, PPW = 64 / LPP, PPB = NW * PPW, H = LG_ATTN_UNIT_H;
    __shared__ float s_o[NW][HD];
    __shared__ float s_m[NW], s_l[NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gl = lane % LPP, grp = lane / LPP;
    /* unit of this workgroup */
    const int blk = blockIdx.x / (8 * NREP), rem = blockIdx.x % (8 * NREP);
    const int r = rem / 8, gc = blk * 8 + rem % 8;
    if (gc >= n_kv * nch) return;   /* padding of the last 8-block: no unit */
    const int c = gc / n_kv, g = gc % n_kv, h = g * NREP + r;
    const int kv_dim = n_kv * HD;
    const int t0 = c * chunk, t1 = min(t0 + chunk, pos + 1);
    const int nsteps = (t1 - t0 + PPB - 1) / PPB;
    const int tcache = min(t1, pos);   /* positions [t0, tcache) come from the cache */

    /* this lane's dims of q_h, and of this step's k and v (used at t == pos) */
    const float4 q0 = *(const float4*)(q + (size_t)h * HD + gl * 8);
    const float4 q1 = *(const float4*)(q + (size_t)h * HD + gl * 8 + 4);
    const float4 k0 = *(const float4*)(kcur + (size_t)g * HD + gl * 8);
    const float4 k1 = *(const float4*)(kcur + (size_t)g * HD + gl * 8 + 4);
    const float4 v0 = *(const float4*)(vcur + (size_t)g * HD + gl * 8);
    const float4 v1 = *(const float4*)(vcur + (size_t)g * HD + gl * 8 + 4);
    uint4 kb[2][H], vb[2][H];
    /* steps sb.. into batch b; rows outside [t0, tcache) load row t0 (unused) */
    auto issue = [&](int b, int sb) {
#pragma unroll
        for (int st = 0; st < H; st++) {
            int t = t0 + (sb + st) * PPB + wave * PPW + grp;
            t = t < tcache ? t : t0;
            const size_t o = (size_t)t * kv_dim + (size_t)g * HD + gl * 8;
            kb[b][st] = *(const uint4*)(kc + o);
            vb[b][st] = *(const uint4*)(vc + o);
        }
    };
    issue(0, 0);
    issue(1, H);
    const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const float kn[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float vn[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;
    /* one online-softmax step of the lane group on the row (k, v) */
    auto step = [&](const float* kf, const float* vf, bool use) {
        float sc = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) sc = __builtin_fmaf(kf[d], qv[d], sc);
        sc = lg_group_sum<LPP>(sc) * scale2;
        if (use) {
            const float mn = fmaxf(m, sc);
            const float a = __builtin_amdgcn_exp2f(m - mn);   /* 0 while m = -inf */
            const float p = __builtin_amdgcn_exp2f(sc - mn);
            l = __builtin_fmaf(l, a, p);
#pragma unroll
            for (int d = 0; d < 8; d++) o[d] = lg_fma2(o[d], a, p, vf[d]);
            m = mn;
        }
    };
    auto process = [&](int b, int sb) {
#pragma unroll
        for (int st = 0; st < H; st++) {
            if (sb + st < nsteps) {   /* uniform over the wave */
                const int t = t0 + (sb + st) * PPB + wave * PPW + grp;
                AttnH8 kh, vh;
                kh.set(kb[b][st]);
                vh.set(vb[b][st]);
                float kf[8], vf[8];
#pragma unroll
                for (int d = 0; d < 8; d++) { kf[d] = kh.f(d); vf[d] = vh.f(d); }
                step(kf, vf, t < tcache);
            }
        }
    };
    /* the loads stay unconditional (past the chunk: row t0 again, unused),
     * so the waits before each batch count only the batches issued before it */
    for (int sb = 0; sb < nsteps; sb += 2 * H) {
        process(0, sb);
        issue(0, sb + 2 * H);
        process(1, sb + H);
        issue(1, sb + 3 * H);
    }
    /* position pos (in the last chunk): this step's fp32 k and v, on lane
     * group 0 of wave 0 */
    if (pos < t1 && wave == 0) step(kn, vn, grp == 0);
    /* the wave's position groups (lanes with the same dims) merge */
    if constexpr (LPP == 8) {
        float o2[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o2[i] = attn_dpp_ror8(o[i]);
        attn_osm_merge(m, l, o, attn_dpp_ror8(m), attn_dpp_ror8(l), o2);
    }
    if constexpr (LPP <= 16) {
        float o2[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o2[i] = lg_partner<4>(o[i]);
        attn_osm_merge(m, l, o, lg_partner<4>(m), lg_partner<4>(l), o2);
    }
    {
        float o2[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o2[i] = lg_partner<5>(o[i]);
        attn_osm_merge(m, l, o, lg_partner<5>(m), lg_partner<5>(l), o2);
    }
    if (grp == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) s_o[wave][gl * 8 + i] = o[i];
        if (gl == 0) { s_m[wave] = m; s_l[wave] = l; }
    }
    attn_bar();
    /* the unit's partial: [m, l, o[HD]] */
    float* part = ws + ((size_t)h * nch + c) * (HD + 2);
    for (int d = tid; d < HD; d += NW * 64) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, s_m[w]);
        float O = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float wt = s_m[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w] - M);
            O = __builtin_fmaf(s_o[w][d], wt, O);
            L = __builtin_fmaf(s_l[w], wt, L);
        }
        part[2 + d] = O;
        if (d == 0) { part[0] = M; part[1] = L; }
    }
}

/* one workgroup per query head: the unit partials [m, l, o[HD]] of its
 * nch chunks merged (weights 2^(m_c - M), as k_attn_merge) */
template <int HD>
__global__ __launch_bounds__(256) void k_attn_unit_merge(const float* __restrict__ ws, int nch, float* __restrict__ out)
{
    __shared__ float s_cm[LG_ATTN_UNIT_MAX_NCH], s_cl[LG_ATTN_UNIT_MAX_NCH];
    const int h = blockIdx.x, tid = threadIdx.x;
    const float* base = ws + (size_t)h * nch * (HD + 2);
    if (tid < nch) { s_cm[tid] = base[(size_t)tid * (HD + 2)]; s_cl[tid] = base[(size_t)tid * (HD + 2) + 1]; }
    __syncthreads();
    float M = -INFINITY;
    for (int cc = 0; cc < nch; cc++) M = fmaxf(M, s_cm[cc]);
    float L = 0.0f;
    for (int cc = 0; cc < nch; cc++) L = __builtin_fmaf(s_cl[cc], __builtin_amdgcn_exp2f(s_cm[cc] - M), L);
    for (int d = tid; d < HD; d += 256) {
        float O = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += 16) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = base[(size_t)min(c0 + k, nch - 1) * (HD + 2) + 2 + d];
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (c0 + k < nch) O = __builtin_fmaf(v[k], __builtin_amdgcn_exp2f(s_cm[c0 + k] - M), O);
        }
        out[(size_t)h * HD + d] = O / L;
    }
}

/* chunking of the unit kernel: 8 chunks up to 512 positions (at least one
 * step each), then a chunk per 256 positions (16 at LG_ATTN_UNIT_CTX) */
static void attn_unit_split(int ctx, int ppb, int* chunk, int* nch)
{
    int n = ctx <= 512 ? 8 : (ctx + 255) / 256;
    if (n > LG_ATTN_UNIT_MAX_NCH) n = LG_ATTN_UNIT_MAX_NCH;
    int c = (ctx + n - 1) / n;
    c = (c + ppb - 1) / ppb * ppb;
    *chunk = c;
    *nch = (ctx + c - 1) / c;
}

template <int HD, int NREP, int LPP>
static void launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                        int n_kv_heads, int pos, float* out, float* ws, hipStream_t s)
{
    const int ctx = pos + 1;
    const float scale = 1.0f / sqrtf((float)HD);
    int ch, nch;
    if constexpr (HD == 64 || HD == 128 || HD == 256) {
        if (pos > 0 && ctx <= LG_ATTN_UNIT_CTX) {
            constexpr int PPB = 4 * (64 / (HD / 8));
            attn_unit_split(ctx, PPB, &ch, &nch);
            const int grid = (n_kv_heads * nch + 7) / 8 * 8 * NREP;
            hipLaunchKernelGGL((k_attn_unit<HD, NREP>), dim3(grid), dim3(256), 0, s, q, k, v, kc, vc, n_kv_heads, pos,
                               ch, nch, scale * 1.44269504088896341f, ws);
            hipLaunchKernelGGL((k_attn_unit_merge<HD>), dim3(n_kv_heads * NREP), dim3(256), 0, s, ws, nch, out);
            return;
        }
        if (attn_tiled(HD, pos)) {
            attn_tile_split(ctx, HD, NREP, &ch, &nch);
            hipLaunchKernelGGL((k_attn_tile<HD, NREP>), dim3(nch, n_kv_heads), dim3(LG_ATTN_TW * 64), 0, s, q, k, v, kc, vc,
                               n_kv_heads * HD, pos, ch, nch, scale * 1.44269504088896341f, ws);
            hipLaunchKernelGGL((k_attn_merge<HD, NREP>), dim3(n_kv_heads * NREP), dim3(256), 0, s, ws, nch, out);
            return;
        }
    }
    ch = attn_chunk(ctx);
    nch = (ctx + ch - 1) / ch;
    hipLaunchKernelGGL((k_attn_split<HD, NREP, LPP>), dim3(nch, n_kv_heads), dim3(256), 0, s, q, k, v, kc, vc,
                       n_kv_heads * HD, pos, ch, nch, scale, ws);
    hipLaunchKernelGGL((k_attn_merge<HD, NREP>), dim3(n_kv_heads * NREP), dim3(256), 0, s, ws, nch, out);
}

template <int HD, int LPP>
static int attn_nrep(int nrep, const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                     int n_kv_heads, int pos, float* out, float* ws, hipStream_t s)
{
    switch (nrep) {
    case 1: launch_attn<HD, 1, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 2: launch_attn<HD, 2, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 4: launch_attn<HD, 4, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 8: launch_attn<HD, 8, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 3: launch_attn<HD, 3, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 5: launch_attn<HD, 5, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 6: launch_attn<HD, 6, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    case 7: launch_attn<HD, 7, LPP>(q, k, v, kc, vc, n_kv_heads, pos, out, ws, s); return 0;
    default: lg_set_error("attention: %d query heads per KV head unsupported (1 to 8)", nrep); return LG_ERR_ARG;
    }
}

int lg_launch_attn(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                   int n_heads, int n_kv_heads, int head_dim, int pos, float* out, void* ws, size_t ws_bytes,
                   hipStream_t s)
{
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || pos < 0 || !q || !k || !v || !out || !ws ||
        (pos > 0 && (!kc || !vc))) {
        lg_set_error("attention: bad arguments (heads %d/%d, pos %d)", n_heads, n_kv_heads, pos);
        return LG_ERR_ARG;
    }
    if (ws_bytes < lg_attn_ws_bytes(n_heads, head_dim, pos)) {
        lg_set_error("attention: workspace of %zu bytes, %zu needed", ws_bytes, lg_attn_ws_bytes(n_heads, head_dim, pos));
        return LG_ERR_ARG;
    }
    const int nrep = n_heads / n_kv_heads;
    float* w = (float*)ws;
    int rc;
    switch (head_dim) {
    case 48: rc = attn_nrep<48, 8>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 64: rc = attn_nrep<64, 8>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 128: rc = attn_nrep<128, 16>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    case 256: rc = attn_nrep<256, 32>(nrep, q, k, v, kc, vc, n_kv_heads, pos, out, w, s); break;
    default: lg_set_error("attention: head_dim %d unsupported (48, 64, 128, 256)", head_dim); return LG_ERR_ARG;
    }
    if (rc) return rc;
    return lg_check_launch("attention");
}

/* ------------------------------------------------------------------ */
/* lg_attn_decode_noalloc: the same kernels on a scratch area that the */
/* library holds in device memory for the life of the process          */
/* ------------------------------------------------------------------ */
/* 8 MiB per device: lg_attn_ws_bytes for 32 heads of 128 up to position
 * 2064383 (504 chunks of 4096 keys), 64 heads of 256 up to 520191 (127
 * chunks).  Every partial is written before it is read, so nothing needs
 * clearing between calls. */
#define LG_ATTN_SCRATCH_BYTES ((size_t)8 << 20)
#define LG_ATTN_SCRATCH_DEVICES 64

static __device__ __align__(256) float scratch[LG_ATTN_SCRATCH_BYTES / sizeof(float)];

/* the device address of `scratch` on each device, looked up once per device
 * with that device current: by lg_create for its device, else by the entry
 * point's first call there; host code passes only these addresses to
 * kernels */
static void* g_scratch_dev[LG_ATTN_SCRATCH_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_device(int* dev)
{
    LG_HIP_CHECK(hipGetDevice(dev));
    if (*dev < 0 || *dev >= LG_ATTN_SCRATCH_DEVICES) {
        lg_set_error("attention scratch: device %d beyond the %d supported", *dev, LG_ATTN_SCRATCH_DEVICES);
        return LG_ERR_ARG;
    }
    return LG_OK;
}

/* looks up the current device's scratch address (once per device) */
int lg_attn_scratch_setup(void)
{
    int dev = 0;
    const int rc = scratch_device(&dev);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            lg_set_error("attention scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
            return LG_ERR_HIP;
        }
        g_scratch_dev[dev] = p;
    }
    return LG_OK;
}

/* the current device's scratch address; the lookup is not made while the
 * stream is being captured into a graph */
static int attn_scratch(hipStream_t stream, void** out)
{
    int dev = 0;
    int rc = scratch_device(&dev);
    if (rc) return rc;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        *out = g_scratch_dev[dev];
    }
    if (*out) return LG_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    LG_HIP_CHECK(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone) {
        lg_set_error("attention (no allocation): the scratch area of device %d is not set up; create a context on "
                     "it (lg_create) or make one call outside graph capture first", dev);
        return LG_ERR_STATE;
    }
    if ((rc = lg_attn_scratch_setup())) return rc;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    *out = g_scratch_dev[dev];
    return LG_OK;
}

extern "C" size_t lg_attn_scratch_bytes(void) { return LG_ATTN_SCRATCH_BYTES; }

extern "C" int lg_attn_decode_noalloc(const float* q, const float* k, const float* v, const uint16_t* kc,
                                      const uint16_t* vc, int n_heads, int n_kv_heads, int head_dim, int pos,
                                      float* out, void* stream)
{
    const size_t need = lg_attn_ws_bytes(n_heads, head_dim, pos);
    if (need > LG_ATTN_SCRATCH_BYTES) {
        lg_set_error("attention (no allocation): %zu bytes of partials needed for %d heads of %d at position %d, "
                     "the scratch area holds %zu", need, n_heads, head_dim, pos, LG_ATTN_SCRATCH_BYTES);
        return LG_ERR_ARG;
    }
    void* ws = nullptr;
    const int rc = attn_scratch((hipStream_t)stream, &ws);
    if (rc) return rc;
    return lg_launch_attn(q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos, out, ws, LG_ATTN_SCRATCH_BYTES,
                          (hipStream_t)stream);
}
