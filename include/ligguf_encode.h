/* ligguf_encode.h -- host-side weight encoders (fp32 -> GGUF block formats)
 * and seeded synthetic tensors.  libligguf_encode.so, plain C + OpenMP.
 *
 * No counterpart in the reference: it reads GGUF blocks (fast/lil_gguf.h:64-113)
 * but ships no weight quantizers.  These encoders write exactly the layouts
 * its dequantizers read (fast/lil_math.cpp:93-298).
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gguf_type numbering (fast/lil_gguf.h:26-43) */
enum {
    LGE_F32 = 0, LGE_F16 = 1, LGE_Q8_0 = 8, LGE_Q2_K = 10, LGE_Q3_K = 11, LGE_Q4_K = 12,
    LGE_Q5_K = 13, LGE_Q6_K = 14, LGE_Q1_0 = 40, LGE_Q1_G = 41
};

/* bytes per row of n values, -1 if n does not fit the block size */
int64_t lge_row_size(int type, int64_t n);

/* out[i] = sigma * N(0,1) drawn from the counter (seed, stream, i) */
void lge_fill_normal(uint64_t seed, uint64_t stream, float* out, int64_t n, float sigma);

/* encode rows x cols floats into rows * lge_row_size(type, cols) bytes */
int lge_quantize(int type, const float* x, int64_t rows, int64_t cols, void* out);

/* encode sigma*N(0,1) values drawn from (seed, stream, r*cols+c) without
 * materialising the fp32 tensor */
int lge_random_tensor(int type, uint64_t seed, uint64_t stream, int64_t rows, int64_t cols, float sigma, void* out);

/* Q1_0 / Q1_G tensors with Bernoulli(0.5) sign bits and |N(0,sigma)| fp16
 * group scales */
int lge_random_q1(int type, uint64_t seed, uint64_t stream, int64_t rows, int64_t cols, float sigma, void* out);

#ifdef __cplusplus
}
#endif
