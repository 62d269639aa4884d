/* Top-p / top-k sampling of a device logits vector (sampler_topp,
 * fast/ligguf_fast_qk.cpp:172-214), so that a sampled decode loop needs no
 * logits copy to the host.
 *
 * The reference: p_i = expf((l_i - max) / temp) (inv_temp = 1 / temp,
 * :178-186), normalised by their sum (:189), sorted by p descending, ties by
 * token ascending (qsort with cmp_sampler_ent_desc, :162-170, :190); top =
 * topp, or p of the first entry when topp <= 0, at most 1 (:192-194); the
 * cutoff is the first index whose cumulative p reaches top, at most topk - 1
 * (:195-204); r = rand() / RAND_MAX * cum (:206) selects the first entry
 * whose cumulative p reaches r (:207-213).  temp <= 0 and a sum <= 0 give the
 * greedy token (:176, :188).
 *
 * Nothing is sorted here.  Every question the sampler asks about the sorted
 * order -- where the running sum first reaches top, which entry has rank
 * topk - 1, where the running sum first reaches r, which token is the j-th
 * of equal p -- is a selection: the 32-bit pattern of a non-negative float
 * orders as the float does, so the entry is found digit by digit (9, 11 and
 * 10 bits: p <= 1 leaves 512 leading values) with histograms of the entries
 * whose higher digits match the prefix chosen so far, each bucket holding a
 * count and the bucket's probability mass.  The mass is summed in 44-bit
 * fixed point with integer atomics, so every sum is the same whatever order
 * the atomics land in.
 *
 * Two launches.  The step is a chain of dependent grid-wide results (max,
 * sum, histogram, choice), and every trip of one through global memory costs
 * about 2 us on MI355X, so the chain is kept short:
 *   max     per block of 256: first-index argmax and the sum of
 *           expf((l - block max) / temp); clears the leading-digit histogram
 *   select  per block of 512 over 2048 entries: the global max and sum
 *           (block sums rescaled), p = expf((l - max) / temp) / sum, the
 *           leading digit's histogram (LDS, then integer atomics), and the
 *           block's entries (pattern, token) written in leading-digit order
 *           with the offset of every digit.  The last block to finish
 *           chooses both cutoff rules' leading digit and, from the bounds the
 *           cutoff bucket puts on the running sum, the range of leading
 *           digits the draw can land in; it gathers those buckets' entries
 *           (every block's slice of them) into LDS and finishes every
 *           selection there: the cutoff's two remaining digits, r, the
 *           pick's three digits, the tie among equal p (the j-th smallest
 *           token: the same selection over the complemented token).  When the
 *           buckets hold more entries than LDS, the selections read the
 *           slices from global memory instead.
 * Fixed-point sums are within 1e-9 of exact: the sampled token is the
 * reference's except where r or top lies within float rounding of a
 * cumulative sum (the reference sums sequentially in float). */
#include <stdint.h>

#include "lg_common.h"

#define LG_SMP_T1 256               /* threads per block, max pass */
#define LG_SMP_MAXB1 1024           /* blocks of the max pass (grid-stride past) */
#define LG_SMP_T2 512               /* threads per block, select pass */
#define LG_SMP_E2 4                 /* entries per thread of the select pass */
#define LG_SMP_R (LG_SMP_T2 * LG_SMP_E2)
#define LG_SMP_MAXB2 1024           /* select blocks: vocabularies up to 2M entries */
#define LG_SMP_FX 44                /* fixed-point fraction bits of the probability mass */
#define LG_SMP_H0 512               /* leading-digit buckets: pattern >> 21 of p in [0, 1] */
#define LG_SMP_NB 2048              /* buckets of the widest later digit (11 bits) */
#define LG_SMP_CAP 12288            /* gathered entries held in LDS */

static_assert(LG_SMP_T2 == LG_SMP_H0, "one leading-digit bucket per thread of the select pass");

/* one selection target: the running-sum (mass) or rank (count) position to
 * find, and what the digits chosen so far leave above it */
struct SmpTarget {
    uint64_t need;          /* mass (fixed point) or count to reach, counted from the top */
    uint64_t mass_above;    /* mass of the entries sorted before the prefix's bucket */
    uint64_t count_above;
    uint32_t prefix;        /* the digits chosen so far */
    int active;             /* 0: this target is not asked */
    int by_count;           /* 1: rank target, 0: mass target */
    int pad_;
};

struct LgSampleWs {
    int n;
    int nb1, nb2;
    float* bmax;            /* [LG_SMP_MAXB1] block max, first index, sum of expf((l - block max) / temp) */
    int* bidx;
    float* bsum;
    uint32_t* h0c;          /* [LG_SMP_H0] leading-digit histogram: counts, masses */
    uint64_t* h0m;
    uint64_t* ent;          /* [nb2][LG_SMP_R] pattern | token << 32, each block's in leading-digit order */
    uint32_t* boff;         /* [nb2][LG_SMP_H0 + 1] offset of each leading digit in the block's entries */
    uint32_t* ctr;          /* [4] last-block counter */
    uint32_t* ready;        /* [nb2] the launch's epoch once the block's entries are stored */
    uint32_t epoch;         /* launches so far (host side) */
    int* out;               /* [1] device */
    int* out_host;          /* [1] pinned host word (its device alias), written with out */
    int* out_host_ptr;      /* the same word, host address */
};

/* (v, i) better than (w, j): larger, or equal and earlier (strict > scan of
 * sampler_greedy, fast/ligguf_fast_qk.cpp:146-160) */
__device__ __forceinline__ bool smp_better(float v, int i, float w, int j)
{
    return v > w || (v == w && i < j);
}

template <int NT>
__device__ __forceinline__ void smp_block_argmax(float& v, int& i)
{
    __shared__ float sv[NT / 64];
    __shared__ int si[NT / 64];
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o);
        const int j = __shfl_xor(i, o);
        if (smp_better(w, j, v, i)) { v = w; i = j; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int k = 1; k < NT / 64; k++)
        if (smp_better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
    __syncthreads();
}

template <int NT, typename T>
__device__ __forceinline__ T smp_block_sum(T v)
{
    __shared__ T ss[NT / 64];
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) ss[wave] = v;
    __syncthreads();
    T s = ss[0];
    for (int k = 1; k < NT / 64; k++) s += ss[k];
    __syncthreads();
    return s;
}

/* exclusive prefix of v over the block's threads in thread order, and the total */
template <int NT, typename T>
__device__ __forceinline__ T smp_block_excl(T v, T* total)
{
    __shared__ T sw[NT / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T incl = v;
    for (int o = 1; o < 64; o <<= 1) {
        const T w = __shfl_up(incl, o);
        if (lane >= o) incl += w;
    }
    if (lane == 63) sw[wave] = incl;
    __syncthreads();
    T pre = 0, all = 0;
    for (int k = 0; k < NT / 64; k++) {
        if (k < wave) pre += sw[k];
        all += sw[k];
    }
    __syncthreads();
    *total = all;
    return pre + incl - v;
}

__device__ __forceinline__ uint64_t smp_fx(float p)
{
    return (uint64_t)((double)p * (double)(1ull << LG_SMP_FX));
}

/* the leading digit of p's pattern (p in [0, 1]; a NaN from NaN logits is
 * kept inside the histogram) */
__device__ __forceinline__ int smp_d0(uint32_t key)
{
    const uint32_t d = key >> 21;
    return d < LG_SMP_H0 ? (int)d : LG_SMP_H0 - 1;
}

/* values other blocks of the running pass wrote: coherent loads */
template <typename T>
__device__ __forceinline__ T smp_ld(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ void smp_st(T* p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* this block's global stores and atomics acknowledged (write-through stores
 * and atomics are then visible to coherent loads anywhere on the device) */
__device__ __forceinline__ void smp_wait_stores()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

/* Is this block the last of the grid to get here?  Every block's atomics and
 * write-through stores before the call are then visible to the last one's
 * coherent loads (the persistent decode kernel's publish protocol: no L2
 * write-back is needed, none of the data goes through it). */
__device__ __forceinline__ bool smp_last_block(uint32_t* ctr)
{
    __shared__ int last;
    smp_wait_stores();
    if (threadIdx.x == 0) last = atomicAdd(ctr, 1u) == gridDim.x - 1;
    __syncthreads();
    return last != 0;
}

/* A histogram scanned in sorted order (largest digit first): thread k holds
 * positions k*per .. k*per+per-1 (position q is bucket nbk-1-q), their
 * counts and masses, and what the positions before them hold. */
struct SmpScan {
    uint64_t m[4], c[4];
    uint64_t em, ec;        /* mass, count at the positions before this thread's */
    uint64_t tm, tc;        /* totals */
    int bits, lp;           /* per = 1 << lp */
};

template <int NT>
__device__ __forceinline__ void smp_scan(const uint32_t* hc, const uint64_t* hm, int bits, SmpScan& S)
{
    __shared__ uint64_t sw[2][NT / 64];
    const int nbk = 1 << bits;
    S.bits = bits;
    S.lp = nbk >= 4 * NT ? 2 : nbk >= 2 * NT ? 1 : 0;
    const int per = 1 << S.lp;
    uint64_t vm = 0, vc = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int pos = threadIdx.x * per + q;
        const bool in = q < per && pos < nbk;
        S.m[q] = in ? hm[nbk - 1 - pos] : 0ull;
        S.c[q] = in ? (uint64_t)hc[nbk - 1 - pos] : 0ull;
        vm += S.m[q];
        vc += S.c[q];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t im = vm, ic = vc;
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t wm = __shfl_up(im, o), wc = __shfl_up(ic, o);
        if (lane >= o) { im += wm; ic += wc; }
    }
    if (lane == 63) { sw[0][wave] = im; sw[1][wave] = ic; }
    __syncthreads();
    uint64_t pm = 0, pc = 0, am = 0, ac = 0;
    for (int k = 0; k < NT / 64; k++) {
        if (k < wave) { pm += sw[0][k]; pc += sw[1][k]; }
        am += sw[0][k];
        ac += sw[1][k];
    }
    __syncthreads();
    S.em = pm + im - vm;
    S.ec = pc + ic - vc;
    S.tm = am;
    S.tc = ac;
}

/* Whole block, target in LDS: the bucket holding the target's position in a
 * scanned histogram: the first non-empty bucket whose running value (count,
 * or mass) reaches the target's remaining need.  Past the last entry (a need
 * beyond the total, e.g. a top that float rounding keeps the sum below) the
 * lowest non-empty bucket is taken: the cutoff rule's "at most the last
 * entry".  The running values only grow, so the threads holding a bucket that
 * reaches the need are all threads from some point on that hold a non-empty
 * bucket: the first of them (one ballot per wave) holds the answer, appends
 * the digit to the prefix and adds what lies above it. */
template <int NT>
__device__ __forceinline__ void smp_find(const SmpScan& S, SmpTarget& tg)
{
    constexpr int NW = NT / 64;
    __shared__ uint64_t s_bf[NW], s_bl[NW];
    const int per = 1 << S.lp;
    const bool byc = tg.by_count != 0;
    const uint64_t above = byc ? tg.count_above : tg.mass_above;
    const uint64_t need = tg.need > above ? tg.need - above : 0ull;
    const bool within = need <= (byc ? S.tc : S.tm);
    uint64_t rm = S.em, rc = S.ec;
    int fq = -1, lq = -1;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (q < per && S.c[q]) {
            const uint64_t inc = byc ? rc + S.c[q] : rm + S.m[q];
            if (fq < 0 && inc >= need) fq = q;
            lq = q;
        }
        rm += S.m[q];
        rc += S.c[q];
    }
    const uint64_t bf = __ballot(fq >= 0), bl = __ballot(lq >= 0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { s_bf[wave] = bf; s_bl[wave] = bl; }
    __syncthreads();
    int owner = -1;
    bool by_first = false;
    if (within)
        for (int w = 0; w < NW && owner < 0; w++)
            if (s_bf[w]) { owner = w * 64 + __ffsll((unsigned long long)s_bf[w]) - 1; by_first = true; }
    for (int w = NW - 1; w >= 0 && owner < 0; w--)
        if (s_bl[w]) owner = w * 64 + 63 - __clzll((long long)s_bl[w]);
    if ((int)threadIdx.x == owner) {
        const int q = by_first ? fq : lq;
        uint64_t am = S.em, ac = S.ec;
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (u < q) { am += S.m[u]; ac += S.c[u]; }
        const int pos = owner * per + q;
        tg.prefix = (tg.prefix << S.bits) | (uint32_t)((1 << S.bits) - 1 - pos);
        tg.mass_above += am;
        tg.count_above += ac;
    }
    __syncthreads();
}

/* entries with pattern `key`: the rank j among them (token order) of the
 * target.  Equal p means equal fixed-point mass P, so the running sum at the
 * j-th of them is mass_above + (j + 1) P. */
__device__ __forceinline__ uint64_t smp_tie_rank(const SmpTarget& t, uint64_t n_eq, uint64_t P)
{
    uint64_t j;
    if (t.by_count) j = t.need - 1 - t.count_above;
    else if (t.need <= t.mass_above + P) j = 0;
    else if (P == 0) j = n_eq - 1;
    else j = (t.need - t.mass_above + P - 1) / P - 1;
    return j < n_eq ? j : n_eq - 1;
}

/* The gathered entries: every block's slice of the leading digits [dl, dh]
 * and of digit bc (when below dl), in LDS (key, idx) or, when they do not
 * fit, read from the blocks' entries each time. */
struct SmpSet {
    const uint32_t* key;    /* LDS copies */
    const uint32_t* idx;
    const uint32_t* s1;     /* per block: start and length of both slices, first gathered position */
    const uint32_t* l1;
    const uint32_t* s2;
    const uint32_t* l2;
    const uint32_t* dst;
    const uint64_t* ent;
    int nb;
    int x;                  /* entries */
    int glob;               /* 1: read from ent */
};

/* every entry of the set's slices in global memory: f(key, idx, position) */
template <int NT, typename F>
__device__ __forceinline__ void smp_each_global(const SmpSet& S, F f)
{
    const int nb = S.nb;
    const int k = nb <= NT ? NT / nb : 1;
    for (int b = nb <= NT ? (int)threadIdx.x / k : (int)threadIdx.x; b < nb; b += nb <= NT ? nb : NT) {
        const int sub = nb <= NT ? (int)threadIdx.x % k : 0;
        const uint32_t n1 = S.l1[b], L = n1 + S.l2[b], a1 = S.s1[b], a2 = S.s2[b], d = S.dst[b];
        const uint64_t* e = S.ent + (size_t)b * LG_SMP_R;
        for (uint32_t i0 = (uint32_t)sub; i0 < L; i0 += 4u * (uint32_t)k) {
            uint64_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t i = i0 + (uint32_t)(u * k);
                v[u] = i < L ? smp_ld(&e[i < n1 ? a1 + i : a2 + (i - n1)]) : 0ull;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t i = i0 + (uint32_t)(u * k);
                if (i < L) f((uint32_t)v[u], (uint32_t)(v[u] >> 32), d + i);
            }
        }
        if (nb <= NT) break;
    }
}

template <int NT, typename F>
__device__ __forceinline__ void smp_each(const SmpSet& S, F f)
{
    if (S.glob) smp_each_global<NT>(S, [&](uint32_t key, uint32_t idx, uint32_t) { f(key, idx); });
    else
        for (int i = threadIdx.x; i < S.x; i += NT) f(S.key[i], S.idx[i]);
}

/* Whole block: histogram (LDS) of one digit (bits at sh) of the set's entries
 * whose higher bits match `prefix`.  by_tok: the digit is of the complemented
 * token (ascending tokens sort first) among the entries whose pattern is K,
 * counts only; else of the pattern, with masses. */
template <int NT>
__device__ __forceinline__ void smp_hist(const SmpSet& S, bool by_tok, uint32_t K, uint32_t prefix, int sh, int bits,
                                         uint32_t* hc, uint64_t* hm)
{
    const int nbk = 1 << bits;
    const uint32_t mask = (uint32_t)nbk - 1u;
    const int hi = sh + bits;
    __syncthreads();   /* the previous readers of hc are done */
    for (int i = threadIdx.x; i < nbk; i += NT) { hc[i] = 0u; hm[i] = 0ull; }
    __syncthreads();
    smp_each<NT>(S, [&](uint32_t key, uint32_t idx) {
        const uint32_t k2 = by_tok ? ~idx : key;
        if ((hi >= 32 || (k2 >> hi) == prefix) && (!by_tok || key == K)) {
            const uint32_t d = (k2 >> sh) & mask;
            atomicAdd(&hc[d], 1u);
            if (!by_tok) atomicAdd((unsigned long long*)&hm[d], (unsigned long long)smp_fx(__uint_as_float(key)));
        }
    });
    __syncthreads();
}

/* Whole block: the target's last two pattern digits (its leading digit is
 * chosen); returns its rank among the entries with its pattern */
template <int NT>
__device__ __forceinline__ uint64_t smp_select_rest(const SmpSet& S, SmpTarget& tg, uint32_t* hc, uint64_t* hm)
{
    SmpScan sc;
    smp_hist<NT>(S, false, 0u, tg.prefix, 10, 11, hc, hm);
    smp_scan<NT>(hc, hm, 11, sc);
    smp_find<NT>(sc, tg);
    smp_hist<NT>(S, false, 0u, tg.prefix, 0, 10, hc, hm);
    smp_scan<NT>(hc, hm, 10, sc);
    smp_find<NT>(sc, tg);
    const uint32_t key = tg.prefix;
    return smp_tie_rank(tg, hc[key & 1023u], smp_fx(__uint_as_float(key)));
}

/* Whole block: the j-th smallest token among the entries whose pattern is K */
template <int NT>
__device__ __forceinline__ uint32_t smp_tie_token(const SmpSet& S, uint32_t K, uint64_t j, uint32_t* hc, uint64_t* hm,
                                                  SmpTarget& tg)
{
    __shared__ uint32_t s_min;
    if (j == 0) {
        __syncthreads();
        if (threadIdx.x == 0) s_min = 0xffffffffu;
        __syncthreads();
        uint32_t mn = 0xffffffffu;
        smp_each<NT>(S, [&](uint32_t key, uint32_t idx) {
            if (key == K && idx < mn) mn = idx;
        });
        for (int o = 32; o > 0; o >>= 1) mn = min(mn, (uint32_t)__shfl_xor((int)mn, o));
        if ((threadIdx.x & 63) == 0 && mn != 0xffffffffu) atomicMin(&s_min, mn);
        __syncthreads();
        return s_min;
    }
    if (threadIdx.x == 0) {
        tg = SmpTarget{};
        tg.need = j + 1;
        tg.by_count = 1;
        tg.active = 1;
    }
    SmpScan sc;
    smp_hist<NT>(S, true, K, 0u, 21, 11, hc, hm);
    smp_scan<NT>(hc, hm, 11, sc);
    smp_find<NT>(sc, tg);
    smp_hist<NT>(S, true, K, tg.prefix, 10, 11, hc, hm);
    smp_scan<NT>(hc, hm, 11, sc);
    smp_find<NT>(sc, tg);
    smp_hist<NT>(S, true, K, tg.prefix, 0, 10, hc, hm);
    smp_scan<NT>(hc, hm, 10, sc);
    smp_find<NT>(sc, tg);
    return ~tg.prefix;
}

/* ------------------------------------------------------------------ */
/* passes                                                               */
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(LG_SMP_T1) void k_smp_max(const float* __restrict__ x, LgSampleWs ws, float inv_temp)
{
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < LG_SMP_H0; i += LG_SMP_T1) { ws.h0c[i] = 0u; ws.h0m[i] = 0ull; }
        if (threadIdx.x < 4) ws.ctr[threadIdx.x] = 0u;
    }
    float v = -INFINITY;
    int i = 0x7fffffff;
    for (int j = blockIdx.x * LG_SMP_T1 + threadIdx.x; j < ws.n; j += gridDim.x * LG_SMP_T1)
        if (smp_better(x[j], j, v, i)) { v = x[j]; i = j; }
    smp_block_argmax<LG_SMP_T1>(v, i);
    /* the block's sum relative to its own max; the select pass rescales it */
    float s = 0.0f;
    if (v != -INFINITY)
        for (int j = blockIdx.x * LG_SMP_T1 + threadIdx.x; j < ws.n; j += gridDim.x * LG_SMP_T1)
            s += expf((x[j] - v) * inv_temp);
    s = smp_block_sum<LG_SMP_T1, float>(s);
    if (threadIdx.x == 0) { ws.bmax[blockIdx.x] = v; ws.bidx[blockIdx.x] = i; ws.bsum[blockIdx.x] = s; }
}

__global__ __launch_bounds__(LG_SMP_T2) void k_smp_select(const float* __restrict__ x, LgSampleWs ws, float inv_temp,
                                                          float topp, int topk, float r01, uint32_t epoch)
{
    constexpr int NT = LG_SMP_T2;
    __shared__ uint32_t s_hc[LG_SMP_NB];
    __shared__ uint64_t s_hm[LG_SMP_NB];
    __shared__ uint32_t s_h0c[LG_SMP_H0];
    __shared__ uint64_t s_h0m[LG_SMP_H0];
    __shared__ uint32_t s_key[LG_SMP_CAP];
    __shared__ uint32_t s_idx[LG_SMP_CAP];
    __shared__ uint32_t s_seg[5][LG_SMP_MAXB2];
    __shared__ SmpTarget s_t[4];
    const int tid = threadIdx.x;
    /* the global max (first index) and the normalising sum, every block alike */
    float M = -INFINITY;
    int mi = 0x7fffffff;
    for (int b = tid; b < ws.nb1; b += NT)
        if (smp_better(ws.bmax[b], ws.bidx[b], M, mi)) { M = ws.bmax[b]; mi = ws.bidx[b]; }
    smp_block_argmax<NT>(M, mi);
    float s = 0.0f;
    for (int b = tid; b < ws.nb1; b += NT)
        if (ws.bmax[b] != -INFINITY) s += ws.bsum[b] * expf((ws.bmax[b] - M) * inv_temp);
    const float sum = smp_block_sum<NT, float>(s);
    if (!(sum > 0.0f)) {
        /* the reference's sum <= 0 case: the greedy token */
        if (blockIdx.x == 0 && tid == 0) { *ws.out = mi; *ws.out_host = mi; }
        return;
    }
    /* p, the leading digit's histogram and each entry's place in its bucket */
    s_h0c[tid] = 0u;
    s_h0m[tid] = 0ull;
    __syncthreads();
    const int lo = blockIdx.x * LG_SMP_R;
    uint32_t key[LG_SMP_E2], pos[LG_SMP_E2];
#pragma unroll
    for (int k = 0; k < LG_SMP_E2; k++) {
        const int j = lo + k * NT + tid;
        key[k] = 0u;
        pos[k] = 0u;
        if (j < ws.n) {
            const float p = expf((x[j] - M) * inv_temp) / sum;
            key[k] = __float_as_uint(p);
            const int d = smp_d0(key[k]);
            pos[k] = atomicAdd(&s_h0c[d], 1u);
            atomicAdd((unsigned long long*)&s_h0m[d], (unsigned long long)smp_fx(p));
        }
    }
    __syncthreads();
    /* the histogram first: the last block starts on it while the entries
     * below are still being stored */
    if (s_h0c[tid]) {
        atomicAdd(&ws.h0c[tid], s_h0c[tid]);
        atomicAdd((unsigned long long*)&ws.h0m[tid], (unsigned long long)s_h0m[tid]);
    }
    const bool last = smp_last_block(ws.ctr);
    uint32_t tot;
    const uint32_t off = smp_block_excl<NT, uint32_t>(s_h0c[tid], &tot);
    s_hc[tid] = off;
    if (tid == 0) s_hc[LG_SMP_H0] = tot;
    __syncthreads();
    uint64_t* ent = ws.ent + (size_t)blockIdx.x * LG_SMP_R;
#pragma unroll
    for (int k = 0; k < LG_SMP_E2; k++) {
        const int j = lo + k * NT + tid;
        if (j < ws.n) smp_st(&ent[s_hc[smp_d0(key[k])] + pos[k]], (uint64_t)key[k] | ((uint64_t)j << 32));
    }
    uint32_t* boff = ws.boff + (size_t)blockIdx.x * (LG_SMP_H0 + 1);
    smp_st(&boff[tid], off);
    if (tid == 0) smp_st(&boff[LG_SMP_H0], tot);
    if (!last) {
        /* publish: every entry acknowledged, then the ready word */
        smp_wait_stores();
        if (tid == 0) smp_st(&ws.ready[blockIdx.x], epoch);
        return;
    }

    /* ---- the last block: every selection ---- */
    s_h0c[tid] = smp_ld(&ws.h0c[tid]);
    s_h0m[tid] = smp_ld(&ws.h0m[tid]);
    if (tid == 0) {
        /* top <= 0: the first entry's own p, reached at rank 0 (mass 1 suffices) */
        const float top = topp > 1.0f ? 1.0f : topp;
        for (int t = 0; t < 4; t++) s_t[t] = SmpTarget{};
        s_t[0].need = top <= 0.0f ? 1ull : smp_fx(top);
        s_t[0].active = 1;
        s_t[1].active = topk > 0 && topk < ws.n;
        s_t[1].by_count = 1;
        s_t[1].need = (uint64_t)(topk > 0 ? topk : 1);
    }
    __syncthreads();
    SmpScan h0;
    smp_scan<NT>(s_h0c, s_h0m, 9, h0);
    smp_find<NT>(h0, s_t[0]);
    if (s_t[1].active) smp_find<NT>(h0, s_t[1]);
    /* the cutoff's bucket: the leading digit sorted first (the larger) */
    const bool c1 = s_t[1].active && s_t[1].prefix > s_t[0].prefix;
    const uint32_t bc = c1 ? s_t[1].prefix : s_t[0].prefix;
    /* the cutoff's running sum lies in (A, A + m]: the draw's need in
     * [floor(r01 A), ceil(r01 (A + m))], whose buckets bound the pick's */
    if (tid == 0) {
        const uint64_t A = c1 ? s_t[1].mass_above : s_t[0].mass_above, m = s_h0m[bc];
        s_t[2].need = (uint64_t)((double)r01 * (double)A);
        const double hi = (double)r01 * (double)(A + m);
        s_t[3].need = (uint64_t)hi + ((double)(uint64_t)hi < hi ? 1 : 0);
    }
    __syncthreads();
    smp_find<NT>(h0, s_t[2]);
    smp_find<NT>(h0, s_t[3]);
    const uint32_t dh = s_t[2].prefix, dl = s_t[3].prefix;
    /* every block's entries stored (this block's own acknowledged too) */
    __shared__ int s_ok;
    smp_wait_stores();
    if (tid < 64) {
        bool ok = false;
        for (int it = 0; !ok && it < (1 << 22); it++) {
            bool mine = true;
            for (int b = tid; b < ws.nb2; b += 64)
                if (b != (int)blockIdx.x && smp_ld(&ws.ready[b]) != epoch) mine = false;
            ok = __all(mine);
        }
        if (tid == 0) s_ok = ok;
    }
    __syncthreads();
    if (!s_ok) {
        /* a block never published (the wait is bounded): no token */
        if (tid == 0) { *ws.out = -1; *ws.out_host = -1; }
        return;
    }
    /* every block's slices of those buckets */
    uint32_t lsum = 0;
    for (int b = tid; b < ws.nb2; b += NT) {
        const uint32_t* bo = ws.boff + (size_t)b * (LG_SMP_H0 + 1);
        const uint32_t a1 = smp_ld(&bo[dl]), e1 = smp_ld(&bo[dh + 1]);
        const bool two = bc < dl;
        const uint32_t a2 = two ? smp_ld(&bo[bc]) : 0u, e2 = two ? smp_ld(&bo[bc + 1]) : 0u;
        s_seg[0][b] = a1;
        s_seg[1][b] = e1 - a1;
        s_seg[2][b] = a2;
        s_seg[3][b] = e2 - a2;
        lsum += e1 - a1 + e2 - a2;
    }
    uint32_t all;
    uint32_t dst = smp_block_excl<NT, uint32_t>(lsum, &all);
    for (int b = tid; b < ws.nb2; b += NT) {
        s_seg[4][b] = dst;
        dst += s_seg[1][b] + s_seg[3][b];
    }
    __syncthreads();
    SmpSet S;
    S.key = s_key;
    S.idx = s_idx;
    S.s1 = s_seg[0];
    S.l1 = s_seg[1];
    S.s2 = s_seg[2];
    S.l2 = s_seg[3];
    S.dst = s_seg[4];
    S.ent = ws.ent;
    S.nb = ws.nb2;
    S.x = (int)all;
    S.glob = all > LG_SMP_CAP;
    if (!S.glob) {
        smp_each_global<NT>(S, [&](uint32_t k, uint32_t i, uint32_t d) {
            s_key[d] = k;
            s_idx[d] = i;
        });
        __syncthreads();
    }
    /* the cutoff: each rule whose entry lies in bucket bc; the first one */
    uint64_t rank0 = ~0ull, rank1 = ~0ull, j0 = 0, j1 = 0;
    if (s_t[0].prefix == bc) {   /* uniform */
        j0 = smp_select_rest<NT>(S, s_t[0], s_hc, s_hm);
        rank0 = s_t[0].count_above + j0;
    }
    if (s_t[1].active && s_t[1].prefix == bc) {
        j1 = smp_select_rest<NT>(S, s_t[1], s_hc, s_hm);
        rank1 = s_t[1].count_above + j1;
    }
    const bool c = rank1 < rank0;
    const SmpTarget& tc = c ? s_t[1] : s_t[0];
    const uint32_t cut_key = tc.prefix;
    const uint64_t cut_j = c ? j1 : j0, cut_rank = c ? rank1 : rank0;
    const uint64_t cum = tc.mass_above + (cut_j + 1) * smp_fx(__uint_as_float(cut_key));
    /* the pick: the first entry whose running sum reaches r (fixed point, rounded up) */
    __syncthreads();
    if (tid == 0) {
        const double rr = (double)r01 * (double)cum;
        uint64_t need = (uint64_t)rr;
        if ((double)need < rr) need++;
        s_t[2] = SmpTarget{};
        s_t[2].need = need;
        s_t[2].active = 1;
    }
    __syncthreads();
    smp_find<NT>(h0, s_t[2]);
    const uint64_t jp = smp_select_rest<NT>(S, s_t[2], s_hc, s_hm);
    uint32_t K = s_t[2].prefix;
    uint64_t jt = jp;
    if (s_t[2].count_above + jp > cut_rank) {
        /* past the cutoff (fixed-point rounding): the cutoff entry */
        K = cut_key;
        jt = cut_j;
    }
    const uint32_t tok = smp_tie_token<NT>(S, K, jt, s_hc, s_hm, s_t[3]);
    if (tid == 0) {
        *ws.out = (int)tok;
        *ws.out_host = (int)tok;
    }
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */
static void smp_free(LgSampleWs* w)
{
    if (!w) return;
    void* bufs[] = {w->bmax, w->bidx, w->bsum, w->h0c, w->h0m, w->ent, w->boff, w->ctr, w->ready, w->out};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (w->out_host_ptr) (void)hipHostFree(w->out_host_ptr);
    delete w;
}

void lg_sample_ws_free(LgSampleWs* w) { smp_free(w); }

int lg_sample_ws_alloc(int n, LgSampleWs** out)
{
    *out = nullptr;
    if (n <= 0 || n > LG_SMP_MAXB2 * LG_SMP_R) {
        lg_set_error("sampler: vocabulary size %d outside 1..%d", n, LG_SMP_MAXB2 * LG_SMP_R);
        return LG_ERR_ARG;
    }
    LgSampleWs* w = new LgSampleWs();
    w->n = n;
    const int nb1 = (n + LG_SMP_T1 * 4 - 1) / (LG_SMP_T1 * 4);
    w->nb1 = nb1 < LG_SMP_MAXB1 ? nb1 : LG_SMP_MAXB1;
    w->nb2 = (n + LG_SMP_R - 1) / LG_SMP_R;
    bool ok = hipMalloc((void**)&w->bmax, LG_SMP_MAXB1 * 4) == hipSuccess &&
              hipMalloc((void**)&w->bidx, LG_SMP_MAXB1 * 4) == hipSuccess &&
              hipMalloc((void**)&w->bsum, LG_SMP_MAXB1 * 4) == hipSuccess &&
              hipMalloc((void**)&w->h0c, LG_SMP_H0 * 4) == hipSuccess &&
              hipMalloc((void**)&w->h0m, LG_SMP_H0 * 8) == hipSuccess &&
              hipMalloc((void**)&w->ent, (size_t)w->nb2 * LG_SMP_R * 8) == hipSuccess &&
              hipMalloc((void**)&w->boff, (size_t)w->nb2 * (LG_SMP_H0 + 1) * 4) == hipSuccess &&
              hipMalloc((void**)&w->ctr, 16) == hipSuccess && hipMalloc((void**)&w->out, 16) == hipSuccess &&
              hipMalloc((void**)&w->ready, (size_t)w->nb2 * 4) == hipSuccess &&
              hipMemset(w->ready, 0, (size_t)w->nb2 * 4) == hipSuccess &&
              hipHostMalloc((void**)&w->out_host_ptr, 64, hipHostMallocDefault) == hipSuccess;
    ok = ok && hipHostGetDevicePointer((void**)&w->out_host, w->out_host_ptr, 0) == hipSuccess;
    if (!ok) {
        smp_free(w);
        lg_set_error("sampler: allocation for %d entries failed", n);
        return LG_ERR_HIP;
    }
    *out = w;
    return LG_OK;
}

int lg_sample_ws_size(const LgSampleWs* w) { return w ? w->n : 0; }

/* the token into ws->out (device) and the pinned host word that
 * lg_sample_ws_out_host returns, valid once the stream has passed the
 * launches; temp > 0 and 0 <= r01 <= 1 checked by the caller */
int lg_launch_sample_topp(const float* logits, LgSampleWs* w, float temp, float topp, int topk, float r01, hipStream_t s)
{
    if (++w->epoch == 0) w->epoch = 1;   /* 0 is the ready words' initial value */
    const LgSampleWs ws = *w;
    const float inv_temp = 1.0f / temp;
    hipLaunchKernelGGL(k_smp_max, dim3(ws.nb1), dim3(LG_SMP_T1), 0, s, logits, ws, inv_temp);
    hipLaunchKernelGGL(k_smp_select, dim3(ws.nb2), dim3(LG_SMP_T2), 0, s, logits, ws, inv_temp, topp, topk, r01,
                       ws.epoch);
    return lg_check_launch("sampler");
}

int* lg_sample_ws_out(LgSampleWs* w) { return w->out; }

int* lg_sample_ws_out_host(LgSampleWs* w) { return w->out_host_ptr; }
