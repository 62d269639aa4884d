/* lg_matvec.hip -- batch-1 quantized matvec for gfx950 (matmul, matmul2,
 * matmul3 of fast/lil_math.cpp:748-899 and the per-format dots of
 * fast/arch_avx2.h:83-435 / fast/lil_math.cpp:396-740).
 *
 * Work split.  A row of n values is cut into "slots" of 64 (K-quants, Q1_G)
 * or 32 (Q8_0, Q1_0, F16, F32) values.  A group of G lanes (G = 64, 32, 16
 * or 8) owns a row; lane j of the group owns slots j, j+G, ... of EVERY row
 * the group visits, so its slice of the quantized activation is loaded once
 * into VGPRs and reused for all rows.  The weight bytes of a slot are read
 * with 128-bit loads straight from the GGUF rows (no repack), RB rows are in
 * flight per group, and the integer sub-block sums run on v_dot4_i32_i8.
 *
 * Numerics.  Per slot the integer sums are exactly the reference's
 * (Notes N2 of the decomposition: sum_g scale_g * sum q*a, minus
 * min_g * bsum_g); they are combined in fp32 per slot and reduced across
 * lanes, so only the fp32 summation order differs from the reference.
 */
#include "lg_common.h"

#include "lg_fmt.h"

/* ------------------------------------------------------------------ */
/* The kernel                                                           */
/* ------------------------------------------------------------------ */
template <int FMT, int G, int NS, int RB>
__global__ __launch_bounds__(256) void k_matvec(const uint8_t* __restrict__ W, uint32_t rsz, int nslots, int d,
                                                const uint8_t* __restrict__ xq, float* __restrict__ y, int accumulate)
{
    using F = Fmt<FMT>;
    constexpr int RPW = 64 / G;
    const int lane = threadIdx.x & 63;
    const int gl = lane & (G - 1);
    const int grp = lane / G;

    typename F::Act act[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int slot = gl + s * G;
        if (slot < nslots) F::load_act(act[s], xq, slot);
    }

    const int gw = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nw = (int)((gridDim.x * blockDim.x) >> 6);
    for (int r0 = gw * RPW * RB; r0 < d; r0 += nw * RPW * RB) {
        typename F::W w[RB][NS];
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const int r = r0 + b * RPW + grp;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const int slot = gl + s * G;
                if (r < d && slot < nslots) F::load_w(w[b][s], W + (size_t)r * rsz, slot);
            }
        }
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const int r = r0 + b * RPW + grp;
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const int slot = gl + s * G;
                if (r < d && slot < nslots) acc += F::dot(w[b][s], act[s], slot);
            }
            acc = lg_group_sum<G>(acc);
            if (gl == 0 && r < d) y[r] = accumulate ? y[r] + acc : acc;
        }
    }
}

/* ------------------------------------------------------------------ */
/* dispatch                                                             */
/* ------------------------------------------------------------------ */
static int vals_per_slot(int type)
{
    switch (type) {
    case LG_Q2_K: case LG_Q3_K: case LG_Q4_K: case LG_Q5_K: case LG_Q6_K: case LG_Q1_G: return 64;
    case LG_Q8_0: case LG_Q1_0: case LG_F16: case LG_F32: return 32;
    default: return 0;
    }
}

template <int FMT, int G, int NS>
static void launch_one(const uint8_t* w, uint32_t rsz, int nslots, int d, const uint8_t* xq, float* y, int acc,
                       hipStream_t s)
{
    constexpr int RB = 2;
    constexpr int rows_per_wave = (64 / G) * RB;
    const int waves = (d + rows_per_wave - 1) / rows_per_wave;
    int blocks = (waves + 3) / 4;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL((k_matvec<FMT, G, NS, RB>), dim3(blocks), dim3(256), 0, s, w, rsz, nslots, d, xq, y, acc);
}

template <int FMT>
static int launch_fmt(const uint8_t* w, uint32_t rsz, int nslots, int d, const uint8_t* xq, float* y, int acc,
                      hipStream_t s)
{
    if (nslots <= 8) { launch_one<FMT, 8, 1>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 16) { launch_one<FMT, 16, 1>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 32) { launch_one<FMT, 16, 2>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 64) { launch_one<FMT, 64, 1>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 128) { launch_one<FMT, 64, 2>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 192) { launch_one<FMT, 64, 3>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 256) { launch_one<FMT, 64, 4>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 384) { launch_one<FMT, 64, 6>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    if (nslots <= 512) { launch_one<FMT, 64, 8>(w, rsz, nslots, d, xq, y, acc, s); return 0; }
    lg_set_error("matvec: row of %d slots exceeds the supported width", nslots);
    return LG_ERR_ARG;
}

int lg_launch_matvec(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, int accumulate,
                     hipStream_t s)
{
    const int64_t need = lg_row_size(type, n);
    const int vps = vals_per_slot(type);
    if (!vps || need < 0) { lg_set_error("matvec: type %d with n=%d unsupported", type, n); return LG_ERR_TYPE; }
    if (!w || !xq || !out || d <= 0 || (int64_t)rsz < need) { lg_set_error("matvec: bad arguments (d=%d rsz=%u need %lld)", d, rsz, (long long)need); return LG_ERR_ARG; }
    if (n % vps) { lg_set_error("matvec: n=%d is not a multiple of %d for type %d", n, vps, type); return LG_ERR_ARG; }
    const int nslots = n / vps;
    const uint8_t* W = (const uint8_t*)w;
    const uint8_t* X = (const uint8_t*)xq;
    int rc;
    switch (type) {
    case LG_Q4_K: rc = launch_fmt<LG_Q4_K>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q5_K: rc = launch_fmt<LG_Q5_K>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q6_K: rc = launch_fmt<LG_Q6_K>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q2_K: rc = launch_fmt<LG_Q2_K>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q3_K: rc = launch_fmt<LG_Q3_K>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q8_0: rc = launch_fmt<LG_Q8_0>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q1_0: rc = launch_fmt<LG_Q1_0>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_Q1_G: rc = launch_fmt<LG_Q1_G>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_F16: rc = launch_fmt<LG_F16>(W, rsz, nslots, d, X, out, accumulate, s); break;
    case LG_F32: rc = launch_fmt<LG_F32>(W, rsz, nslots, d, X, out, accumulate, s); break;
    default: lg_set_error("matvec: type %d unsupported", type); return LG_ERR_TYPE;
    }
    if (rc) return rc;
    return lg_check_launch("matvec");
}
